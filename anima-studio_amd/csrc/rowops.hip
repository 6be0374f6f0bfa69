// Row kernels of the attention sublayer: per-head q/k RMSNorm + RoPE (in place), RMSNorm, RoPE.
// Built with -ffp-contract=off and the reduction order of the reference's shaders, so the fp32
// results are bit-identical to a sequential restatement of app/gpu/kernels.js.
#include <cmath>

#include "common.h"
#include "internal.h"

namespace anima {

// One wave per (token, q-or-k head), 4 per workgroup; lane i owns the RoPE pair (i, i + D/2)
// (app/gpu/kernels.js:314-333).
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(float* X, int64_t L, int H, int D, int64_t ld,
                                                           const float* QN, const float* KN, const float* CS,
                                                           int64_t sin_off, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (id >= L * 2 * H) return;
  const int half = D >> 1;
  const int64_t l = id / (2 * H);
  const int h = (int)(id - l * 2 * H);
  float* base = X + l * ld + (int64_t)h * D;
  float x1 = 0.0f, x2 = 0.0f, red = 0.0f;
  if (lane < half) {
    x1 = base[lane];
    x2 = base[lane + half];
    red = x1 * x1 + x2 * x2;
  }
  red = tree_sum_down(red, half);
  const float total = __shfl(red, 0);
  const float r = 1.0f / sqrtf(total / (float)D + eps);
  if (lane < half) {
    const float* w = h < H ? QN : KN;
    const float y1 = x1 * r * w[lane];
    const float y2 = x2 * r * w[lane + half];
    const float c = CS[l * half + lane];
    const float s = CS[sin_off + l * half + lane];
    base[lane] = y1 * c - y2 * s;
    base[lane + half] = y2 * c + y1 * s;
  }
}

// One wave per row, 4 rows per workgroup: 64 strided partial sums then a 32..1 tree
// (app/gpu/kernels.js:73-88).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* X, const float* W, float* Y, int64_t rows,
                                                      int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* x = X + row * cols;
  float ss = 0.0f;
  for (int c = lane; c < cols; c += 64) ss += x[c] * x[c];
  ss = tree_sum_down(ss, 64);
  const float r = 1.0f / sqrtf(__shfl(ss, 0) / (float)cols + eps);
  float* y = Y + row * cols;
  for (int c = lane; c < cols; c += 64) y[c] = x[c] * r * W[c];
}

// One thread per rotated pair (app/gpu/kernels.js:343-356).
__global__ __launch_bounds__(256) void rope_kernel(float* X, const float* CS, int64_t L, int H, int D,
                                                   int64_t sin_off, int64_t row_stride, int64_t col_off) {
  const int half = D >> 1;
  const int64_t n = L * H * half;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * 256) {
    const int i = (int)(idx % half);
    const int h = (int)((idx / half) % H);
    const int64_t l = idx / ((int64_t)half * H);
    float* base = X + l * row_stride + col_off + (int64_t)h * D;
    const float c = CS[l * half + i], s = CS[sin_off + l * half + i];
    const float x1 = base[i], x2 = base[i + half];
    base[i] = x1 * c - x2 * s;
    base[i + half] = x2 * c + x1 * s;
  }
}

int qk_norm_rope_launch(anima_ctx* c, float* qkv, int64_t L, int H, int D, int64_t ld, const float* qn,
                        const float* kn, const float* cs, int64_t sin_off, float eps) {
  if (!qkv || !qn || !kn || !cs) return fail(c, ANIMA_E_ARG, "anima_qk_norm_rope: null pointer");
  if (D != 64 && D != 128) return fail(c, ANIMA_E_UNSUPPORTED, "anima_qk_norm_rope: D=%d (64 or 128)", D);
  if (L < 0 || H < 1 || ld < 2LL * H * D) return fail(c, ANIMA_E_ARG, "anima_qk_norm_rope: L=%lld H=%d ld=%lld (ld >= 2*H*D)", (long long)L, H, (long long)ld);
  if (sin_off < L * (D / 2)) return fail(c, ANIMA_E_ARG, "anima_qk_norm_rope: sin_off=%lld < L*D/2", (long long)sin_off);
  if (L == 0) return ANIMA_OK;
  const int64_t waves = L * 2 * H;
  Launch lc(c, "qk_norm_rope", 0.0, (double)waves * D * 4 * 2 + (double)L * D * 4);
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, c->stream, qkv, L, H, D,
                     ld, qn, kn, cs, sin_off, eps);
  return lc.end();
}

int rmsnorm_launch(anima_ctx* c, const float* x, const float* w, float* y, int64_t rows, int cols, float eps) {
  if (!x || !w || !y) return fail(c, ANIMA_E_ARG, "anima_rmsnorm: null pointer");
  if (rows < 0 || cols < 1) return fail(c, ANIMA_E_ARG, "anima_rmsnorm: rows=%lld cols=%d", (long long)rows, cols);
  if (rows == 0) return ANIMA_OK;
  Launch lc(c, "rmsnorm", 0.0, (double)rows * cols * 8);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, c->stream, x, w, y, rows, cols, eps);
  return lc.end();
}

int rope_launch(anima_ctx* c, float* x, const float* cs, int64_t L, int H, int D, int64_t sin_off,
                int64_t row_stride, int64_t col_off) {
  if (!x || !cs) return fail(c, ANIMA_E_ARG, "anima_rope: null pointer");
  if (D < 2 || D % 2 || H < 1 || L < 0) return fail(c, ANIMA_E_ARG, "anima_rope: L=%lld H=%d D=%d", (long long)L, H, D);
  if (row_stride < col_off + (int64_t)H * D || col_off < 0) return fail(c, ANIMA_E_ARG, "anima_rope: row_stride=%lld col_off=%lld", (long long)row_stride, (long long)col_off);
  if (sin_off < L * (D / 2)) return fail(c, ANIMA_E_ARG, "anima_rope: sin_off=%lld < L*D/2", (long long)sin_off);
  const int64_t n = L * H * (D / 2);
  if (n == 0) return ANIMA_OK;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
  Launch lc(c, "rope", 0.0, (double)n * 16);
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)blocks), dim3(256), 0, c->stream, x, cs, L, H, D, sin_off, row_stride, col_off);
  return lc.end();
}

}  // namespace anima
