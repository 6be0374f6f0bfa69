/*
 * anima.h -- C ABI of the MI355X (gfx950) DiT attention hot path.
 *
 * One context = one HIP device + one HIP stream.  Every compute entry point is enqueued on
 * that stream, returns immediately, and reports errors as a negative status; the message of
 * the last failure is kept per context (anima_last_error).  Arguments are validated on the
 * host before any HIP call.  A context is used from one host thread at a time, like the
 * reference's single-threaded WebGPU runtime (app/gpu/device.js:59-232).
 *
 * Pointers passed to compute entry points are device pointers (from anima_alloc or any HIP
 * allocation on the context's device).  Element offsets, leading dimensions and batch strides
 * are in elements, as in the reference's op layer (app/gpu/ops.js).
 *
 * Citations (file:line) name the reference interface each entry point replaces, relative to
 * the anima-studio repository.
 */
#ifndef ANIMA_H
#define ANIMA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANIMA_OK 0
#define ANIMA_E_ARG (-1)         /* invalid argument (shape, stride, alignment, null) */
#define ANIMA_E_HIP (-2)         /* a HIP runtime call failed */
#define ANIMA_E_OOM (-3)         /* device allocation failed */
#define ANIMA_E_STATE (-4)       /* context lost / unusable after an earlier device error */
#define ANIMA_E_UNSUPPORTED (-5) /* valid request this build does not implement */

typedef struct anima_ctx anima_ctx;

/* ---------------------------------------------------------------- runtime
 * Replaces GPU.create / GPU / BufferPool / Profiler of app/gpu/device.js. */

/* GPU.create (app/gpu/device.js:61-81): bind `device`, create the stream. */
int anima_init(int device, anima_ctx** out);
/* Frees pooled memory, events and the stream (pipeline unload, app/pipeline.js:165-176). */
int anima_destroy(anima_ctx* ctx);
/* Message of the last failed call on ctx (or of anima_init when ctx is NULL). */
const char* anima_last_error(const anima_ctx* ctx);
/* GPU.sync (app/gpu/device.js:218-222): wait for all enqueued work, surface deferred errors. */
int anima_sync(anima_ctx* ctx);
/* GPU.flush (app/gpu/device.js:206-216): work is submitted at enqueue time; a no-op kept for
 * interface parity. */
int anima_flush(anima_ctx* ctx);
/* BufferPool.allocated / peak (app/gpu/device.js:26-57) plus bytes parked in free lists. */
int anima_mem_stats(anima_ctx* ctx, uint64_t* allocated, uint64_t* peak, uint64_t* pooled);
/* The adapter limits of app/gpu/device.js:63-88 (GPU.limits, GPU.maxBinding) for this context's
 * device.  WebGPU caps one buffer and one binding; HIP caps neither below the device memory, so
 * both report the device's global memory, and a caller sizing chunks from them (the score chunks
 * of app/gpu/ops.js:177-181) gets the same bound the library's own chunked path respects
 * (anima_attention: score chunks of at most 1 GiB). */
typedef struct {
  int64_t max_buffer_size;             /* maxBufferSize: the device's global memory */
  int64_t max_binding_size;            /* maxStorageBufferBindingSize: the same */
  int64_t total_memory, free_memory;   /* hipMemGetInfo at the call */
  int32_t workgroup_storage_size;      /* maxComputeWorkgroupStorageSize: LDS bytes per workgroup */
  int32_t max_workgroup_size;          /* maxComputeInvocationsPerWorkgroup */
  int32_t max_workgroups_per_dimension; /* maxComputeWorkgroupsPerDimension (grid x) */
  int32_t compute_units;
  int32_t wavefront_size;
  int32_t clock_khz;                   /* peak shader clock */
  char arch[64];                       /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} anima_limits;
int anima_device_limits(anima_ctx* ctx, anima_limits* out);
/* BufferPool.get (app/gpu/device.js:40-48): device memory from 1/8-power-of-two size buckets. */
int anima_alloc(anima_ctx* ctx, size_t bytes, void** out);
/* Tensor.release / BufferPool.put (app/gpu/device.js:20-23, 49-52): back to its bucket.
 * Reuse is stream-ordered, so work already enqueued on the buffer stays valid. */
int anima_free(anima_ctx* ctx, void* ptr);
/* BufferPool.trim (app/gpu/device.js:53-56): synchronize and release every parked buffer. */
int anima_pool_trim(anima_ctx* ctx);
/* GPU.write / fromArray (app/gpu/device.js:113-131): host -> device, stream-ordered; the host
 * buffer may be reused when the call returns.  Copies up to 4 MiB go through a ring of pinned
 * staging slots and return without waiting for the work already on the stream (as
 * queue.writeBuffer does); larger ones wait for the stream to reach the copy. */
int anima_h2d(anima_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Queue marks, for the reference's periodic `await gpu.sync()` in long encodes
 * (app/pipeline.js:255, every 7 DiT blocks): anima_mark records the current end of the
 * stream and returns its ticket; anima_wait_mark(t) blocks until the work enqueued before mark t
 * has finished and surfaces deferred device errors like anima_sync.  Waiting for the mark before
 * the last one keeps work queued on the device while the host catches up.  Tickets older than
 * the 16 most recent marks wait for a later mark (a superset of their work). */
int anima_mark(anima_ctx* ctx, uint64_t* ticket);
int anima_wait_mark(anima_ctx* ctx, uint64_t ticket);
/* GPU.read (app/gpu/device.js:141-154): device -> host, waits for the stream. */
int anima_d2h(anima_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Device-to-device copy (the copyBufferToBuffer of concatLinears, app/weights.js:168-184). */
int anima_d2d(anima_ctx* ctx, void* dst, const void* src, size_t bytes);

/* Profiler (app/gpu/device.js:234-288): when enabled, every kernel launch is bracketed by HIP
 * events on the context stream and aggregated by kernel name with its algorithmic flops and
 * bytes.  report() synchronizes and writes a JSON array
 * [{"name","count","ms","flops","bytes"}, ...] sorted by time (descending). */
int anima_profile_enable(anima_ctx* ctx, int on);
int anima_profile_reset(anima_ctx* ctx);
int anima_profile_report(anima_ctx* ctx, char* buf, size_t len);
/* Wall time of stream work between two marks (HIP events on the context stream). */
int anima_timer_start(anima_ctx* ctx);
int anima_timer_stop(anima_ctx* ctx, float* ms);

/* ABI self-description, for bindings that restate the descriptor structs below (ctypes, FFI):
 * the byte offset of `field` in the struct named `type` -- "anima_attn_desc", "anima_linear_desc",
 * "anima_weight", "anima_sampler_desc", "anima_conv_desc", "anima_limits", "anima_qkv_desc" -- or the
 * struct's size when `field` is
 * NULL; -1 for a name this library does not know.  No counterpart in the reference (its op layer
 * has no C ABI); it lets a binding refuse to load when its layout differs from the library's. */
int64_t anima_abi_offset(const char* type, const char* field);

/* Recorded submission.  The reference records its dispatches into command encoders and submits
 * them in batches (app/gpu/device.js:1-5, 183-216), re-recording every forward.  Here the
 * context stream's work between anima_graph_begin and anima_graph_end is captured once into a
 * HIP graph and anima_graph_launch replays it (same kernels, same arguments, same device
 * addresses; inputs are read as they are when the replay runs).
 * While capturing, host copies (anima_h2d, anima_d2h) and synchronization (anima_sync,
 * anima_pool_trim, the profiler report, the timer) fail with ANIMA_E_STATE.  Buffers freed during
 * the capture, and the scratch the captured calls are handed (a pool buffer of the size each call
 * asks for, never the context's own workspace), stay reserved for the graph until
 * anima_graph_destroy; buffers still allocated at the end (outputs) and those allocated before
 * the capture (inputs, weights) remain the caller's and must stay allocated while the graph is
 * replayed.  Profiling is suspended during the capture. */
typedef struct anima_graph anima_graph;
int anima_graph_begin(anima_ctx* ctx);
/* Ends the capture; on success *graph is replayable.  On failure the capture is discarded. */
int anima_graph_end(anima_ctx* ctx, anima_graph** graph);
int anima_graph_launch(anima_ctx* ctx, anima_graph* graph);
/* Releases the graph; its reserved buffers go back to the pool (stream-ordered). */
int anima_graph_destroy(anima_ctx* ctx, anima_graph* graph);

/* ---------------------------------------------------------------- attention */

#define ANIMA_PREC_BF16 0 /* bf16 MFMA, fp32 accumulate */
#define ANIMA_PREC_FP32 1 /* fp32 MFMA (tolerance variant) */

typedef struct {
  int B, Lq, Lk, H, D; /* D == 128 and D == 64 (the LLM adapter's heads; operands zero-padded to 128
                        * dims) on the flash kernels, as ops.js:170 sends D in {64, 128} to
                        * flashAttentionShader; other D % 4 == 0 (the VAE's 384) on the chunked path of
                        * app/gpu/ops.js:177-207, causal mask included.  Fused norm / RoPE and
                        * prepared K/V need D == 128 (D == 64 with them takes the chunked path). */
  int group;           /* q heads per kv head (1 = MHA); 0 is read as 1 */
  const float* q;
  int64_t ldq, q_off, q_bstride;
  const float* k;
  int64_t ldk, k_off, k_bstride;
  const float* v;
  int64_t ldv, v_off, v_bstride;
  float* o;
  int64_t ldo, o_off, o_bstride;
  float scale;         /* 0 -> 1/sqrt(D) */
  const int* kv_len;   /* host array [B] of valid key counts in [1, Lk]; NULL -> Lk */
  int precision;       /* ANIMA_PREC_* */
  /* Optional fused per-head RMSNorm (weight [D], eps) + split-half RoPE (table: cos block then
   * sin block, [rows][D/2] each, sin block at rope_sin_off) on the Q and K loads. */
  const float* q_norm;
  const float* k_norm;
  const float* rope_cs;
  int64_t rope_sin_off;
  float eps;
  int causal; /* 1: keys after the query's own index are masked, limit = min(Lk, query + 1)
               * (the causal softmax of app/gpu/kernels.js:27-49, used by the text encoder's
               * attention, app/models/qwen3.js:60); with group > 1 this is its GQA form */
  /* Optional: K and V already converted by anima_attention_prepare_kv (same B, H / group, Lk and
   * precision); then k, v, their strides, k_norm and the key side of rope_cs are not read. */
  const void* kv_prep;
  /* With kv_prep (and for anima_attention_prepare_kv): the prepared buffer's size, which must equal
   * anima_attention_kv_bytes(B, H / group, Lk, precision) -- a buffer prepared for another shape or
   * precision is rejected instead of being read past its end. */
  int64_t kv_prep_bytes;
  /* Optional: Q as anima_linear_qkv's q_prep writes it (bf16 [B][Lq][H][128], the query after
   * q_norm and RoPE times scale * log2(e)); then q, ldq, q_off, q_bstride, q_norm and the query
   * side of rope_cs are not read, and the attention's scale is the one Q was prepared with.  bf16
   * precision and D = 128 only; the results equal those of the fp32 q with q_norm / rope_cs. */
  const void* q_prep;
  /* 1: O is written as bf16 (round to nearest even of the fp32 result; o, o_off, ldo and
   * o_bstride then address uint16 elements, ldo % 4 == 0, o 8-byte aligned): the input of a
   * quantized output projection, which reads it with anima_quant_rows_bf16.  bf16 precision with
   * D = 128 or 64 (the flash kernels) only. */
  int o_bf16;
} anima_attn_desc;

/* ops.attention (app/gpu/ops.js:166-208) on the flash path (kernels.js:158-299), plus the fused
 * q/k RMSNorm + RoPE of ops.qkNormRope (ops.js:140-145) when q_norm/k_norm/rope_cs are set:
 * O[b, i, o_off + h*D + d] = softmax(scale * q_i . k_j, j < kv_len[b]) . v.
 * q/k/v/o element (b, row, head h, dim d) lives at ptr[b*bstride + row*ld + off + h*D + d]
 * (kv head h/group for k and v). */
int anima_attention(anima_ctx* ctx, const anima_attn_desc* desc);
/* The K/V half of anima_attention on its own: K rows RMS-normalized (k_norm) and rotated (rope_cs)
 * and V transposed, rounded to the MFMA operand type, written to kv_prep
 * (anima_attention_kv_bytes(B, H / group, Lk, precision) bytes, passed in desc->kv_prep_bytes,
 * 16-byte aligned) for later
 * anima_attention calls with desc->kv_prep: keys and values that serve many calls (the per-prompt
 * cross-attention K/V of app/models/dit.js:232-249) are converted once. */
int anima_attention_prepare_kv(anima_ctx* ctx, const anima_attn_desc* desc, void* kv_prep);
int64_t anima_attention_kv_bytes(int B, int Hkv, int Lk, int precision);

/* anima_attention without any device allocation.  No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  The same kernels and results as anima_attention (bit-identical); the K/V conversion
 * goes into a static device array of anima_attention_noalloc_scratch_bytes() (64 MiB) per GPU,
 * loaded with the library and held until the process ends, instead of the context's workspace.
 * A call whose K/V conversion needs more (anima_attention_kv_bytes(B, H / group, Lk, precision)
 * above the maximum; B=2, 16 heads, Lk=4096 in bf16 is exactly 64 MiB) fails with ANIMA_E_ARG;
 * with desc->kv_prep set no scratch is used.  D must be 128 (ANIMA_E_UNSUPPORTED otherwise).  The
 * profiler records nothing for these calls.  Every call on one GPU shares that GPU's array: calls
 * on different contexts / streams of the same GPU that overlap in time race on it (serialize them). */
int anima_attention_noalloc(anima_ctx* ctx, const anima_attn_desc* desc);
int64_t anima_attention_noalloc_scratch_bytes(void);

/* ---------------------------------------------------------------- row ops */

/* ops.qkNormRope (app/gpu/ops.js:140-145; kernels.js:304-334): in place on the q and k parts of
 * a fused QKV buffer X[L][ld] (q heads at 0, k heads at H*D). */
int anima_qk_norm_rope(anima_ctx* ctx, float* qkv, int64_t L, int H, int D, int64_t ld,
                       const float* q_norm, const float* k_norm, const float* cs,
                       int64_t sin_off, float eps);
/* ops.rmsnorm (app/gpu/ops.js:111-117; kernels.js:65-89 mode 0). y may equal x. */
int anima_rmsnorm(anima_ctx* ctx, const float* x, const float* w, float* y, int64_t rows,
                  int cols, float eps);
/* ops.rope (app/gpu/ops.js:148-152; kernels.js:337-357): in place on X viewed as [L][H][D]
 * inside rows of row_stride starting at col_off. */
int anima_rope(anima_ctx* ctx, float* x, const float* cs, int64_t L, int H, int D,
               int64_t sin_off, int64_t row_stride, int64_t col_off);

/* ops.rotate (app/gpu/ops.js:38-44; kernels.js:360-388): y = x @ H per contiguous group of 256
 * features, H = kron(H4,H4,H4,H4)/16.  n % 256 == 0; y may equal x. */
int anima_hadamard(anima_ctx* ctx, const float* x, float* y, int64_t n);
/* Per-token dynamic int8 quantization of rows x[M][K] (no reference counterpart: the reference
 * keeps activations fp32).  With rotate != 0 the ConvRot Hadamard of anima_hadamard is applied
 * first (K % 256 == 0).  s[m] = amax_k|x_r[m,k]| / 127 (0 for an all-zero row),
 * q[m,k] = clamp(rint(x_r[m,k] / s[m]), -127, 127).  K % 4 == 0, K <= 8192. */
int anima_quant_rows(anima_ctx* ctx, const float* x, int64_t M, int K, int rotate, int8_t* q,
                     float* s);
/* Splits fp32 src[n] into three bf16 planes dst[3][n]: dst0 = bf16(src), dst1 = bf16(src - dst0),
 * dst2 = bf16(src - dst0 - dst1) (round to nearest even; each difference is exact in fp32), the
 * ANIMA_W_F32S3 layout (no reference counterpart: the load-time form of the LoRA matrices of
 * app/lora.js:103-134).  n % 8 == 0, 16-byte aligned pointers. */
int anima_split3_bf16(anima_ctx* ctx, const float* src, uint16_t* dst, int64_t n);
/* anima_quant_rows of act(x) (ANIMA_ACT_*, the epilogue activations of anima_linear, the same
 * functions): a linear that feeds a quantized linear can store its pre-activation output and
 * leave the activation to this pass (the MLP's GELU between mlp.layer1 and mlp.layer2,
 * app/models/dit.js:306-311).  The int8 rows equal those of anima_quant_rows on the stored
 * activation output. */
int anima_quant_rows_act(anima_ctx* ctx, const float* x, int64_t M, int K, int act, int rotate,
                         int8_t* q, float* s);
/* anima_quant_rows of bf16 rows (each value widened exactly to fp32 first: the same int8 rows and
 * scales as anima_quant_rows on the widened rows): the attention output written with
 * anima_attn_desc.o_bf16.  K = 1024, 2048, 4096 or 8192; x and q 16-byte aligned. */
int anima_quant_rows_bf16(anima_ctx* ctx, const uint16_t* x, int64_t M, int K, int rotate, int8_t* q, float* s);
/* ops.layernormMod (app/gpu/ops.js:129-137; kernels.js:95-145): LayerNorm without affine,
 * y = LN(x) * (1 + mod[scale_off + c]) + mod[shift_off + c], then the ConvRot Hadamard when
 * rotate != 0.  Writes the fp32 result to y (if non-NULL) and/or its per-token int8
 * quantization to q, s (if non-NULL; requires rotate).  cols % 256 == 0 when rotating,
 * cols <= 8192. */
int anima_layernorm_mod(anima_ctx* ctx, const float* x, const float* mod, int64_t shift_off,
                        int64_t scale_off, int64_t rows, int cols, float eps, int rotate, float* y,
                        int8_t* q, float* s);

#define ANIMA_EW_SILU_MUL 0 /* y = silu(a) * b */
#define ANIMA_EW_ADD 1      /* y = a + b */
#define ANIMA_EW_SILU 2     /* y = silu(a) */
#define ANIMA_EW_COPY 3     /* y = a */
/* ops.elementwise (app/gpu/ops.js:154-160; kernels.js:391-413). */
int anima_elementwise(anima_ctx* ctx, int op, const float* a, const float* b, float* y, int64_t n);
/* ops.zero (app/gpu/ops.js:89-93; kernels.js:415-423). */
int anima_zero(anima_ctx* ctx, float* y, int64_t n);

/* patchify on the device (app/models/dit.js:55-65, a host loop in the reference): latents
 * [B][16][h][w] -> patches [B*(h/2)*(w/2)][68], "c (h m) (w n) -> (h w) (c m n)", columns 64..67
 * (the padding-mask channel) zero.  h, w even. */
int anima_patchify(anima_ctx* ctx, const float* latents, int B, int h, int w, float* patches);
/* unpatchify on the device (app/models/dit.js:68-78): final-layer output [B*(h/2)*(w/2)][64] in
 * (p1 p2 c) order -> latents [B][16][h][w], "(h w) (p1 p2 c) -> c (h p1) (w p2)".  h, w even. */
int anima_unpatchify(anima_ctx* ctx, const float* o, int B, int h, int w, float* latents);

/* One sampler step on the device, replacing the host loops of app/pipeline.js:276-283 (CFG
 * combine v = vu + cfg (vc - vu), denoised = x - sigma v) and of app/samplers.js:104-218 (the
 * per-sampler update of x).  Every value the reference stores into a Float32Array is formed here
 * in double precision from the same operands in the same order, without fused multiply-adds, and
 * rounded to float at the same point, so that on equal inputs x, den, old and old_d are
 * bit-identical to the reference's.  The scalar coefficients c[] are computed by the host exactly
 * as the reference computes them (see each kind):
 *   EULER     c0 = s1/s, c1 = 1 - s1/s:                      x = c0 x + c1 den
 *   EULER_A   c0 = r, c1 = 1 - r, c2 = k, c3 = renoise:       t = c0 x + c1 den; x = c2 t + eps c3
 *   DPMPP_2M  c0 = ratio, c1 = -expm1(-h); stage 1 adds c2 = 1 + 1/(2 r), c3 = -1/(2 r):
 *             dd = stage ? c2 den + c3 old : den;             x = c0 x + c1 dd
 *   ER_SDE    c0 = (alpha_t / alpha_s) r, c1 = alpha_t (1 - r): x = c0 x + c1 den; stage >= 2:
 *             c2, c3 = +-1/(l_s - l_{i-1}), c4: dD = c2 den + c3 old, x = x + c4 dD, old_d = dD;
 *             stage 3: c5, c6 = +-2/(l_s - l_{i-2}), c7: dU = c5 dD + c6 old_d, x = x + c7 dU;
 *             eps != NULL: c8 = alpha_t, c9 = nz: x = x + (c8 eps) c9
 * final_step != 0 (next sigma 0): x = den.  old (DPMPP_2M, ER_SDE) is read when needed and then
 * overwritten with den; den_out (optional) receives den. */
#define ANIMA_SAMPLER_EULER 0
#define ANIMA_SAMPLER_EULER_A 1
#define ANIMA_SAMPLER_DPMPP_2M 2
#define ANIMA_SAMPLER_ER_SDE 3
typedef struct anima_sampler_desc {
  int kind;
  int64_t n;             /* latent elements of one image */
  float* x;              /* [n] in / out */
  const float* v;        /* [n] velocity of the (positive) conditioning */
  const float* v_uncond; /* [n] velocity of the negative prompt, NULL without CFG */
  double cfg;
  double sigma;
  int final_step;        /* next sigma is 0 */
  int stage;             /* DPMPP_2M: 0 first step, 1 later; ER_SDE: 1, 2 or 3 */
  float* den_out;        /* [n] or NULL */
  float* old;            /* [n] previous den (DPMPP_2M, ER_SDE), else NULL */
  float* old_d;          /* [n] previous first difference (ER_SDE), else NULL */
  const float* eps;      /* [n] noise (EULER_A, ER_SDE) or NULL */
  double c[10];
} anima_sampler_desc;
int anima_sampler_step(anima_ctx* ctx, const anima_sampler_desc* d);

/* Seeded synthetic data on the device, for benchmarks and tests (no reference counterpart: the
 * reference loads real checkpoints).  Element i draws h = splitmix64(seed * 0xD1B54A32D192ED03 + i):
 *   ANIMA_FILL_U8    uint8   lo + h % (hi - lo + 1)                (integers lo..hi)
 *   ANIMA_FILL_I8N   int8    clamp(((b0+b1+b2+b3 - 510) * round(lo * 4096 / 147.8017)) >> 12, +-127)
 *                            (b_j = bytes of h: Irwin-Hall approximation of N(0, lo^2))
 *   ANIMA_FILL_F32   fp32    lo + (hi - lo) * ((h >> 40) * 2^-24)
 *   ANIMA_FILL_BF16  bf16    the ANIMA_FILL_F32 value rounded to nearest even
 *   ANIMA_FILL_F32N  fp32    (u0+u1+u2+u3 - 2) * 1.7320508 * lo + hi, u_j = 16-bit fields of h / 65536 */
#define ANIMA_FILL_U8 0
#define ANIMA_FILL_I8N 1
#define ANIMA_FILL_F32 2
#define ANIMA_FILL_BF16 3
#define ANIMA_FILL_F32N 4
int anima_fill_random(anima_ctx* ctx, void* dst, int64_t n, int kind, uint64_t seed, float lo, float hi);

/* ---------------------------------------------------------------- VAE decoder ops */

/* ops.conv3x3 / conv3x3Into (app/gpu/ops.js:95-109; the implicit-GEMM "conv3" loader of
 * app/gpu/gemm.js:56-80): out[b][y][x][n] (+)= bias[n] + sum_{tap, ci} w[n][tap][ci] * in(b, y + ty - 1,
 * x + tx - 1, ci), zero padding, NHWC fp32 activations, bf16 OHWI weights [cout][3][3][cin] (the
 * checkpoint layout of tools/build_assets.py:160-180).  up = 1 reads the input through a 2x nearest
 * upsample: in(b, y, x) = x_in[b][y/2][x/2], the input being H/2 x W/2.  precision: ANIMA_PREC_FP32
 * keeps fp32-level accuracy (activations as two bf16 terms on the bf16 matrix cores), ANIMA_PREC_BF16
 * rounds them to bf16.  cin % 16 == 0; x and w 16-byte aligned. */
typedef struct {
  int B, H, W;       /* images and output size */
  int cin, cout;
  int up;
  const float* x;    /* [B][H or H/2][W or W/2][cin] */
  const uint16_t* w; /* [cout][9 * cin] */
  const float* bias; /* [cout] or NULL */
  float* out;        /* [B][H][W][cout] */
  int resid;         /* 1: out += conv (conv3x3Into) */
  int precision;
} anima_conv_desc;
int anima_conv3x3(anima_ctx* ctx, const anima_conv_desc* desc);
/* ops.channelNorm (app/gpu/ops.js:119-126; kernels.js:62-89 mode 1, the Wan VAE RMS_norm):
 * y = x * sqrt(cols) / max(||x||, 1e-12) * gamma per row, then SiLU when silu != 0.  y may equal x. */
int anima_channel_norm(anima_ctx* ctx, const float* x, const float* gamma, float* y, int64_t rows, int cols, int silu);
/* The decoder's image conversion (app/models/vae.js:104-112, a host loop in the reference) on the
 * device: out[i] = RGBA bytes of x[i][0..2], each round((clamp(v, -1, 1) + 1) / 2 * 255) with the
 * reference's double-precision arithmetic and Math.round ties; alpha 255.  out 4-byte aligned. */
int anima_to_rgba(anima_ctx* ctx, const float* x, int64_t n, uint8_t* out);

/* ---------------------------------------------------------------- linears */

#define ANIMA_W_BF16 0 /* bf16 [N][K]; fp32 activations, fp32 accumulation (gemm.js:108-128) */
#define ANIMA_W_I8 1   /* int8 [N][K] + weight_scale [N] (comfy_quant int8_tensorwise+convrot) */
#define ANIMA_W_W4 2   /* 4-bit codes [N][K/2] (low nibble = even k) + s_rel e4m3 [N][K/16] +
                          s_channel [N] + codebook [16] (comfy_quant asym_w4a8_int8+convrot) */
#define ANIMA_W_F32 3  /* fp32 [N][K]; fp32 activations, fp32 accumulation: the LoRA A / B matrices
                          of app/lora.js:103-134, run by ops.js:70-87 as kind "f32" */
#define ANIMA_W_F32S3 4 /* an fp32 [N][K] matrix as three bf16 planes [3][N][K] (anima_split3_bf16:
                           w = w0 + w1 + w2 to within 2^-24 |w|); the product runs on the bf16 matrix
                           cores as sum_{i+j<=2} x_i w_j with x split the same way on the fly, fp32
                           accumulation: fp32-level accuracy (not bit-identical to ANIMA_W_F32) at
                           ~1/3 of the fp32 matrix-core time.  K % 8 == 0.  The same LoRA matrices. */
#define ANIMA_ACT_NONE 0
#define ANIMA_ACT_GELU 1 /* erf GELU (kernels.js:9-20) */
#define ANIMA_ACT_SILU 2
#define ANIMA_EPI_STORE 0 /* out = r */
#define ANIMA_EPI_RESID 1 /* out += r */
#define ANIMA_EPI_GATED 2 /* out = fma(gate[gate_off + n], r, out) */

/* Linear weight object of app/weights.js:1-4, 118-147 (device pointers). */
typedef struct {
  int kind, N, K;
  const void* w;
  const float* scale;      /* i8: weight_scale [N]; w4: weight_s_channel [N] */
  const uint8_t* srel;     /* w4: [N][K/16] fp8 e4m3 */
  const float* codebook;   /* w4: [16] */
  const float* bias;       /* [N] or NULL */
} anima_weight;

typedef struct {
  int64_t M;
  const anima_weight* W;
  /* fp32 input x[M][ldx].  For i8/w4 weights the input must be ConvRot-rotated: x_rotated = 1
   * means x already is (ops.linear's opts.xr), 0 rotates it here (ops.js:52-54). */
  const float* x;
  int64_t ldx;
  int x_rotated;
  /* i8/w4: pre-quantized rotated activations (anima_quant_rows / anima_layernorm_mod); when set,
   * x is ignored.  f32s3 (split) weights take them in place of x as well (x NULL; K % 16 == 0,
   * ldx % 16 == 0 in bytes, xq 16-byte aligned): y = xs[m] * sum_k xq[m][k] W[n][k], the LoRA A
   * product of a quantized linear over the int8 rows its GEMM reads, with the rotated A. */
  const int8_t* xq;
  const float* xs;
  float* out;
  int64_t ldc;   /* 0 -> N */
  float alpha;   /* 0 -> 1 */
  int act;       /* ANIMA_ACT_* */
  int epilogue;  /* ANIMA_EPI_* */
  const float* gate;
  int64_t gate_off;
  int32_t* acc_out; /* i8/w4 only, optional: the raw int32 accumulators [M][N] */
  /* optional fp32 term add[m*ld_add + n] added after the bias and before the activation: the ADD
   * input of gemm.js:189 that carries the LoRA delta of ops.js:55-62 (ld_add 0 -> N) */
  const float* add;
  int64_t ld_add;
  /* i8/w4 only, optional: the LoRA delta of ops.js:55-62 (sum over entries of scale * B (A x_in))
   * computed inside the epilogue from its two factors instead of passed as `add`:
   * y += sum_k lora_xa[m*ld_lora_xa + k] * B[n][k] for k < lora_r, after the bias and before the
   * activation / gate, with lora_xa the A products (fp32 [M][ld_lora_xa]) and lora_b the three
   * bf16 planes [3][N][lora_r] (anima_split3_bf16) of B, every entry's scale folded into its
   * columns.  lora_r % 16 == 0, ld_lora_xa % 4 == 0, both 16-byte aligned; not with `add`.
   * lora_cols > 0: block-diagonal ranks (a stacked q/k/v projection whose parts carry their own
   * LoRAs): column n takes the lora_r ranks of its block, lora_xa columns (n / lora_cols) *
   * lora_r + k, so lora_b is [3][N][lora_r] with only the block's own ranks; N % lora_cols == 0,
   * lora_cols % 16 == 0, ld_lora_xa >= (N / lora_cols) * lora_r.  0: one block over all N. */
  const float* lora_xa;
  int64_t ld_lora_xa;
  const uint16_t* lora_b;
  int lora_r;
  int lora_cols;
} anima_linear_desc;

/* ops.linear (app/gpu/ops.js:48-66) -> matmulShader (gemm.js:166-280):
 * r = alpha * (x @ dec(W)^T); i8/w4: dec is the int8 grid and r is scaled by s_x[m] * s_w[n]
 * (W8A8: activations quantized per token after the ConvRot rotation); then + bias[n], act,
 * and the store / residual / gated-residual epilogue of gemm.js:186-192.
 * i8/w4 need K % 64 == 0 (and K <= 8192 when x is quantized here). */
int anima_linear(anima_ctx* ctx, const anima_linear_desc* desc);

/* The stacked QKV projection of a DiT block with the attention's operand preparation in its
 * epilogue: app/models/dit.js:266-304 runs ops.linear (qkv), ops.qkNormRope (q and k in place) and
 * the flash attention, whose operands this library converts first (anima_attention_prepare_kv).
 * Here the GEMM that produces qkv writes, per token,
 *   Q  columns [0, 128 H)        fp32 into d->out (row stride d->ldc >= 128 H), as anima_linear,
 *                                or with q_prep the attention's prepared bf16 Q (below);
 *   K  columns [128 H, 256 H)    RMSNorm(k_norm, eps) + RoPE (rope_cs, as anima_attn_desc), bf16,
 *   V  columns [256 H, 384 H)    bf16, transposed,
 * K and V into kv_prep in the layout of anima_attention_prepare_kv(B, Lq = Lk = L, H heads,
 * bf16) -- the same bytes, bit for bit, as preparing this linear's fp32 output -- for
 * anima_attention(desc->kv_prep = kv_prep) with q = d->out, q_norm and the same RoPE table.
 * Requirements: int8 or W4 weights with N = 3 * 128 * H (H even; or 128 * H with q_prep), the
 * store epilogue (bias and alpha allowed; no activation, add term or acc_out; the LoRA factors of
 * anima_linear_desc with rank blocks of whole 256-column tiles), M = B * L with L % 64 == 0,
 * 16-byte aligned buffers; ANIMA_E_UNSUPPORTED otherwise (the caller then runs anima_linear +
 * anima_attention). */
typedef struct {
  int B, L, H;          /* batch elements, tokens each (M = B * L), heads of 128 */
  const float* k_norm;  /* [128] */
  const float* rope_cs; /* cos block [rows][64] then sin block at rope_sin_off, rows >= L */
  int64_t rope_sin_off;
  float eps;
  void* kv_prep;        /* anima_attention_kv_bytes(B, H, L, ANIMA_PREC_BF16) bytes */
  int64_t kv_prep_bytes;
  /* Optional: Q in the attention's prepared form (anima_attn_desc.q_prep) instead of fp32 into
   * out: B * L * H * 128 bf16 values, each the attention's own bf16(scale * log2(e) * q') of the
   * query q' after q_norm (if given) and RoPE (if rope_cs is given); q_scale 0 -> 1 / sqrt(128).
   * With q_prep, N may also be H * 128 (a Q-only projection: no K / V, kv_prep and k_norm unused,
   * rope_cs optional). */
  const float* q_norm;
  void* q_prep;
  float q_scale;
} anima_qkv_desc;
int anima_linear_qkv(anima_ctx* ctx, const anima_linear_desc* desc, const anima_qkv_desc* qkv);

/* The int8 grid of a W4 weight, grid[n][k] = clamp(rint(codebook[code] * fp8(s_rel)), -127, 127)
 * for the 4-bit code of (n, k): the values gemm.js:141-158's W4 B-loader multiplies
 * (tools/quant.py:127-129).  An i8 weight {grid, scale = the W4 weight's s_channel, bias} then
 * gives bit-identical anima_linear results on the int8 path; a loader that can spend the memory
 * (one byte per weight instead of half a byte) converts W4 weights once at load time this way.
 * grid: [N][K] int8, 16-byte aligned; K % 32 == 0. */
int anima_weight_unpack_w4(anima_ctx* ctx, const anima_weight* w4, int8_t* grid);

/* Where anima_linear / anima_linear_qkv turn a W4 weight's nibbles into int8 grid values on the
 * persistent 256 x 256 GEMM (products with at least one 256 x 256 tile per compute unit; smaller
 * products always unpack inside their GEMM).  No counterpart in the reference, whose W4 B-loader
 * decodes inside the matmul (gemm.js:141-158); both paths give bit-identical results.
 *   ANIMA_W4_GRID_SCRATCH (default): one pass writes the weight's int8 grid (anima_weight_unpack_w4
 *     semantics) into a pooled scratch buffer of N * K bytes, released after the call; the int8
 *     GEMM reads it.  The weight stays packed in memory; the nibble work runs once per call
 *     instead of once per row tile.
 *   ANIMA_W4_IN_GEMM: every workgroup unpacks its B tiles inside the GEMM main loop (no scratch). */
#define ANIMA_W4_GRID_SCRATCH 0
#define ANIMA_W4_IN_GEMM 1
int anima_set_w4_path(anima_ctx* ctx, int path);

/* G independent small-M bf16-weight products in one launch, for the adaLN modulation linears of
 * timeCond (app/models/dit.js:196-225 runs one per block and kind, all on the same sigma):
 *   out[g*out_gstride + m*ldc + n] = sum_k x[g*x_gstride + m*ldx + k] * w[g*w_gstride + n*K + k]
 *                                    (+ bias[g*bias_gstride + n])
 * for g < G, m < M, n < N, with the fp32 FMA order of anima_linear's bf16 GEMV.  M <= 8,
 * K % 8 == 0, x and w 16-byte aligned, ldx and x_gstride multiples of 4, w_gstride of 8; a
 * bias_gstride of 0 adds the same bias to every group. */
int anima_linear_grouped_bf16(anima_ctx* ctx, int G, int64_t M, int N, int K, const float* x, int64_t ldx,
                              int64_t x_gstride, const uint16_t* w, int64_t w_gstride, const float* bias,
                              int64_t bias_gstride, float* out, int64_t ldc, int64_t out_gstride);

/* G independent fp32 GEMVs (one input row each) in one launch, for the LoRA products of the adaLN
 * modulation linears (ops.js:70-87 runs two matmuls per LoRA entry; timeCond has one entry per
 * modulation linear, all of one rank):
 *   y[g*y_gstride + n] = alpha * sum_k w[g*w_gstride + n*K + k] * x[g*x_gstride + k]
 *                        (+ y[g*y_gstride + n] when accumulate)
 * for g < G, n < N, the sum in k order with fp32 FMAs.  K % 4 == 0, x and w 16-byte aligned,
 * x_gstride and w_gstride multiples of 4; alpha 0 means 1. */
int anima_gemv_grouped_f32(anima_ctx* ctx, int G, int N, int K, const float* x, int64_t x_gstride, const float* w,
                           int64_t w_gstride, float* y, int64_t y_gstride, float alpha, int accumulate);

#ifdef __cplusplus
}
#endif
#endif
