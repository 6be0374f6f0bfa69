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
/* BufferPool.get (app/gpu/device.js:40-48): device memory from 1/8-power-of-two size buckets. */
int anima_alloc(anima_ctx* ctx, size_t bytes, void** out);
/* Tensor.release / BufferPool.put (app/gpu/device.js:20-23, 49-52): back to its bucket.
 * Reuse is stream-ordered, so work already enqueued on the buffer stays valid. */
int anima_free(anima_ctx* ctx, void* ptr);
/* BufferPool.trim (app/gpu/device.js:53-56): synchronize and release every parked buffer. */
int anima_pool_trim(anima_ctx* ctx);
/* GPU.write / fromArray (app/gpu/device.js:113-131): host -> device, stream-ordered; the host
 * buffer may be reused when the call returns. */
int anima_h2d(anima_ctx* ctx, void* dst, const void* src, size_t bytes);
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

/* ---------------------------------------------------------------- attention */

#define ANIMA_PREC_BF16 0 /* bf16 MFMA, fp32 accumulate */
#define ANIMA_PREC_FP32 1 /* fp32 MFMA (tolerance variant) */

typedef struct {
  int B, Lq, Lk, H, D; /* D == 128 */
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
  int causal; /* must be 0: the causal chunked path of the text encoder is not on this path */
} anima_attn_desc;

/* ops.attention (app/gpu/ops.js:166-208) on the flash path (kernels.js:158-299), plus the fused
 * q/k RMSNorm + RoPE of ops.qkNormRope (ops.js:140-145) when q_norm/k_norm/rope_cs are set:
 * O[b, i, o_off + h*D + d] = softmax(scale * q_i . k_j, j < kv_len[b]) . v.
 * q/k/v/o element (b, row, head h, dim d) lives at ptr[b*bstride + row*ld + off + h*D + d]
 * (kv head h/group for k and v). */
int anima_attention(anima_ctx* ctx, const anima_attn_desc* desc);

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

#ifdef __cplusplus
}
#endif
#endif
