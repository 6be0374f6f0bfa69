/*
 * CPU oracle for the DiT attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's math, used by tests/, the smoke check and
 * the bench's CPU baseline leg as the checker.  Nothing in the product (libanima.so,
 * the N-API addon, the JS host) links, loads or calls this code.
 *
 * Every function names the reference file:line it follows (paths relative to the
 * anima-studio repository).  Layouts are the reference's: row-major fp32 activations,
 * fused QKV rows [L][3*H*D], RoPE tables as a cos block followed by a sin block.
 *
 * Pinning (what independent check fixes each function) is listed in tests/ and in the
 * design notes; see the per-function comments below for the reference citation.
 */
#ifndef ANIMA_ORACLE_H
#define ANIMA_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* torch.manual_seed(seed); torch.randn(n) on the CPU generator (app/rng.js:5-67). n >= 16. */
void orc_randn(uint64_t seed, int64_t n, float* out);
/* One raw MT19937 draw stream (app/rng.js:5-34), for the generator's own check. */
void orc_mt19937(uint32_t seed, int64_t n, uint32_t* out);

/* 3D Cosmos RoPE angles [Hp*Wp][64] (app/models/common.js:31-52). */
void orc_dit_rope_angles(int Hp, int Wp, float* out);
/* cos block then sin block, each [L][half] (app/models/common.js:3-12). */
void orc_rope_table(const float* angles, int64_t L, int half, float* out);

/* In-place per-head RMSNorm + split-half RoPE on q and k of X[L][ld]
 * (app/gpu/kernels.js:304-334, dispatched by app/gpu/ops.js:140-145). */
void orc_qk_norm_rope(float* X, int64_t L, int H, int D, int64_t ld, const float* qn,
                      const float* kn, const float* cs, int64_t sin_off, float eps);
/* y = x * rsqrt(mean(x^2) + eps) * w over rows of `cols` (app/gpu/kernels.js:65-89, mode 0). */
void orc_rmsnorm(const float* X, const float* W, float* Y, int64_t rows, int cols, float eps);
/* In-place split-half RoPE on X viewed as [L][H][D] (app/gpu/kernels.js:337-357). */
void orc_rope(float* X, const float* cs, int64_t L, int H, int D, int64_t sin_off,
              int64_t row_stride, int64_t col_off);

/* y = x @ H per 256-group, H = kron(H4,H4,H4,H4)/16 (app/gpu/kernels.js:360-388). n % 256 == 0. */
void orc_hadamard256(const float* X, float* Y, int64_t n);
/* LayerNorm (no affine) + adaLN (+ ConvRot Hadamard) (app/gpu/kernels.js:95-145). */
void orc_layernorm_mod(const float* X, const float* MOD, float* Y, int64_t rows, int cols,
                       int64_t shift_off, int64_t scale_off, float eps, int rotate);

/* Attention over strided fp32 views (the addressing of app/gpu/ops.js:166-175).
 * q: row (b*q_bs + i*ldq + q_off + h*D); k/v: row (b*k_bs + j*ldk + k_off + (h/group)*D);
 * o: (b*o_bs + i*ldo + o_off + h*D).  kv_len[b] (NULL: Lk) masks keys >= kv_len[b], which is
 * what the reference kernel does for keys >= Lk (app/gpu/kernels.js:245-247). */
typedef struct {
  int B, Lq, Lk, H, D, group;
  const float *q, *k, *v;
  float* o;
  int64_t ldq, ldk, ldv, ldo, q_off, k_off, v_off, o_off, q_bs, k_bs, v_bs, o_bs;
  float scale;
  const int* kv_len;
} orc_attn;

/* fp64 brute force softmax(scale Q K^T) V (tools/reference.py:109-111 math). */
void orc_attention_f64(const orc_attn* a);
/* fp32 step-by-step restatement of flashAttentionShader (app/gpu/kernels.js:158-299):
 * 64-row x 32-key tiles, key mask -1e30, natural exp, partial-sum order of the shader. */
void orc_attention_wgsl(const orc_attn* a);
/* bf16-MFMA numerics model of this build's kernel: Q*c (c = scale*log2e), K and V rounded to
 * bf16 (round to nearest even), fp32 scores s = bf16(Q c) . bf16(K), p = exp2(s - m) with an
 * integer row offset m, O = sum(bf16(p) * V) / sum(bf16(p)).  (With an integer m the value
 * of m only scales every p by the same power of two; the kernel's lazily raised offset and
 * this row maximum give the same weights.) */
void orc_attention_bf16(const orc_attn* a);

/* bf16 round-to-nearest-even of an fp32 value, returned as fp32. */
float orc_bf16_round(float x);

/* Per-token dynamic int8 quantization (no reference implementation; this build's
 * definition): s = amax/127 (0 if amax == 0), q = clamp(rint(x * (127/amax)), -127, 127)
 * (one fp32 multiply by the rounded inverse, not a division, per element). */
void orc_token_quant(const float* X, int64_t M, int K, int8_t* Q, float* S);
/* acc[m][n] = sum_k qx[m][k] * qw[n][k], exact int32. */
void orc_gemm_i8(const int8_t* QX, const int8_t* QW, int64_t M, int N, int K, int32_t* ACC);
/* fp8 e4m3 -> fp32 (app/gpu/gemm.js:144-151). */
float orc_fp8e4m3(uint8_t b);
/* W4 -> int8 grid: clamp(round_half_even(codebook[c] * fp8(s_rel)), -127, 127)
 * (tools/quant.py:127-129, 172-182; app/gpu/gemm.js:141-158).  codes [N][K/2] with the
 * low nibble = even k (tools/quant.py:162); s_rel [N][K/16]. */
void orc_w4_decode(const uint8_t* codes, const uint8_t* srel, const float* codebook, int N,
                   int K, int8_t* out);
/* Epilogue of matmulShader (app/gpu/gemm.js:186-192) applied to integer accumulators with
 * per-token activation scales: r = (acc * sx[m]) * sw[n] (+bias) (act), then
 * store / C += r / C += gate[g_off+n] * r.  act: 0 none, 1 gelu, 2 silu.
 * epi: 0 store, 1 resid, 2 gated resid.  sx == NULL means 1. */
void orc_linear_epilogue(const int32_t* ACC, int64_t M, int N, const float* sx, const float* sw,
                         const float* bias, int act, int epi, const float* gate, int64_t g_off,
                         float* C, int64_t ldc, const float* add);
/* erf-GELU with Abramowitz-Stegun 7.1.26 (app/gpu/kernels.js:9-20). */
float orc_gelu(float x);
float orc_silu(float x);

/* The seeded synthetic-weight fill of anima_fill_random (include/anima.h; no reference
 * counterpart): element i draws h = splitmix64(seed * 0xD1B54A32D192ED03 + i).  kind: 0 U8,
 * 1 I8N, 2 F32, 3 BF16 (bits), 4 F32N. */
void orc_fill_random(void* dst, int64_t n, int kind, uint64_t seed, float lo, float hi);
/* Wan VAE channel norm (app/gpu/kernels.js:62-89 mode 1): y = x * sqrt(cols) / max(||x||, 1e-12) * g,
 * then SiLU when silu != 0, in the shader's reduction order. */
void orc_channel_norm(const float* X, const float* G, float* Y, int64_t rows, int cols, int silu);
/* splitmix64's output for one state (Vigna's reference generator), for its known-answer check. */
uint64_t orc_splitmix64_next(uint64_t state);

#ifdef __cplusplus
}
#endif
#endif
