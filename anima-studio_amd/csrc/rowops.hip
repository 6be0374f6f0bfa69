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

// In-place 4-stage radix-4 butterfly over each 256-group of S[0..cols) (app/gpu/kernels.js:124-140),
// 256 threads, quads strided over the row.  Caller synchronizes before and after.
__device__ __forceinline__ void butterfly_rows(float* S, int cols) {
  const int t = threadIdx.x;
  const int quads = cols >> 2;
  int stride = 1;
  for (int d = 0; d < 4; d++) {
    for (int q = t; q < quads; q += 256) {
      const int g = q >> 6, w = q & 63;
      const int i0 = g * 256 + (w / stride) * stride * 4 + w % stride;
      const float a = S[i0], b = S[i0 + stride], c = S[i0 + 2 * stride], e = S[i0 + 3 * stride];
      S[i0] = a + b + c - e;
      S[i0 + stride] = a + b - c + e;
      S[i0 + 2 * stride] = a - b + c + e;
      S[i0 + 3 * stride] = -a + b + c + e;
    }
    __syncthreads();
    stride *= 4;
  }
}

// Block-wide reduction in the order of the shaders' "red[t] += red[t + s]" loops (s = 128..1).
__device__ __forceinline__ float block_tree_sum(float v, float* red) {
  const int t = threadIdx.x;
  red[t] = v;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] = red[t] + red[t + s];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return r;
}

// Per-token int8 of the row held in S (256 threads): s = amax/127, q = clamp(rint(x * (127/amax))).
__device__ __forceinline__ void quant_row(const float* S, int cols, float* red, int8_t* q, float* s_out) {
  const int t = threadIdx.x;
  float amax = 0.0f;
  for (int c = t; c < cols; c += 256) amax = fmaxf(amax, fabsf(S[c]));
  amax = block_max(amax, red);
  const float s = amax / 127.0f, inv = 127.0f / amax;
  if (t == 0) *s_out = s;
  for (int c4 = t; c4 < (cols >> 2); c4 += 256) {
    char4 o;
    int8_t* ob = (int8_t*)&o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float v = amax == 0.0f ? 0.0f : rintf(S[4 * c4 + j] * inv);
      v = fminf(fmaxf(v, -127.0f), 127.0f);
      ob[j] = (int8_t)v;
    }
    *(char4*)(q + 4 * c4) = o;
  }
}

// One wave per 256-group (app/gpu/kernels.js:366-388), 4 groups per workgroup.
__global__ __launch_bounds__(256) void hadamard_kernel(const float* X, float* Y, int64_t groups) {
  __shared__ float S[4][256];
  const int w = threadIdx.x >> 6, t = threadIdx.x & 63;
  const int64_t g = (int64_t)blockIdx.x * 4 + w;
  const bool live = g < groups;
  float* s = S[w];
  if (live)
    for (int j = 0; j < 4; j++) s[t + 64 * j] = X[g * 256 + t + 64 * j];
  __syncthreads();
  int stride = 1;
  for (int d = 0; d < 4; d++) {
    const int lo = t % stride;
    const int i0 = (t / stride) * stride * 4 + lo;
    const float a = s[i0], b = s[i0 + stride], c = s[i0 + 2 * stride], e = s[i0 + 3 * stride];
    __syncthreads();
    s[i0] = a + b + c - e;
    s[i0 + stride] = a + b - c + e;
    s[i0 + 2 * stride] = a - b + c + e;
    s[i0 + 3 * stride] = -a + b + c + e;
    __syncthreads();
    stride *= 4;
  }
  if (live)
    for (int j = 0; j < 4; j++) Y[g * 256 + t + 64 * j] = s[t + 64 * j] * 0.0625f;
}

// LayerNorm (no affine) + adaLN modulation (+ Hadamard) (+ int8), one workgroup per row
// (app/gpu/kernels.js:108-145); used for rows over 2048 columns and when the rows or the
// modulation vectors are not 16-byte aligned (the wave-per-row kernel below reads float4s).
__global__ __launch_bounds__(256) void layernorm_mod_kernel(const float* X, const float* MOD, int64_t shift_off,
                                                            int64_t scale_off, int cols, float eps, int rotate, float* Y,
                                                            int8_t* Q, float* S_out) {
  extern __shared__ float S[];
  __shared__ float red[256];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* x = X + row * cols;
  float s = 0.0f;
  for (int c = t; c < cols; c += 256) s += x[c];
  const float mean = block_tree_sum(s, red) / (float)cols;
  float v = 0.0f;
  for (int c = t; c < cols; c += 256) {
    const float d = x[c] - mean;
    v += d * d;
  }
  const float r = 1.0f / sqrtf(block_tree_sum(v, red) / (float)cols + eps);
  for (int c = t; c < cols; c += 256) S[c] = (x[c] - mean) * r * (1.0f + MOD[scale_off + c]) + MOD[shift_off + c];
  __syncthreads();
  if (rotate) {
    butterfly_rows(S, cols);
    for (int c = t; c < cols; c += 256) S[c] = S[c] * 0.0625f;
    __syncthreads();
  }
  if (Y)
    for (int c = t; c < cols; c += 256) Y[row * cols + c] = S[c];
  if (Q) quant_row(S, cols, red, Q + row * cols, S_out + row);
}

// ------------------------------------------------------------------ conflict-free row variants
//
// The row lives in LDS with 4 floats of padding after every 64 (element p at p + 4*(p/64)).
// Butterfly stage 1 (stride 1) is done in registers on the float4 chunks as they are loaded;
// stages 2-4 go through LDS, and with the padding every access of those stages is free of bank
// conflicts: stride 4 and stride 64 keep the natural quad order, stride 16 gives lane
// (16a + m) the quad m of 64-block 4a + c (c = 0..3 per pass), so the 64 lanes of an
// instruction hit 64 distinct banks.  T = 64 * WPR threads work on one row (WPR waves; one wave
// needs no barriers because a wave's own LDS accesses complete in issue order).
__device__ __forceinline__ int padx(int p) { return p + 4 * (p >> 6); }

__device__ __forceinline__ float4 bfly4(float4 v) {
  return make_float4(v.x + v.y + v.z - v.w, v.x + v.y - v.z + v.w, v.x - v.y + v.z + v.w, -v.x + v.y + v.z + v.w);
}

template <int WPR>
__device__ __forceinline__ void row_sync() {
  if constexpr (WPR > 1) __syncthreads();
}

// Stages 2-4 over the padded row S (stage 1 already applied), T = 64*WPR threads, thread tr.
template <int WPR>
__device__ __forceinline__ void butterfly_stages234(float* S, int cols, int tr) {
  constexpr int T = 64 * WPR;
  const int quads = cols >> 2;
  // stride 4: quad w -> elements 16(w/4) + w%4 + 4k
  for (int w = tr; w < quads; w += T) {
    const int i0 = 16 * (w >> 2) + (w & 3);
    const float a = S[padx(i0)], b = S[padx(i0 + 4)], c = S[padx(i0 + 8)], e = S[padx(i0 + 12)];
    S[padx(i0)] = a + b + c - e;
    S[padx(i0 + 4)] = a + b - c + e;
    S[padx(i0 + 8)] = a - b + c + e;
    S[padx(i0 + 12)] = -a + b + c + e;
  }
  row_sync<WPR>();
  // stride 16: thread (wave wv, lane 16a + m) -> quad m of 64-block 4a + c + 16 (wv + WPR i)
  {
    const int wv = tr >> 6, aa = (tr >> 4) & 3, mm = tr & 15;
    const int nblk = cols >> 6;
    for (int base = 16 * wv; base < nblk; base += 16 * WPR)
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int blk = base + 4 * aa + c;
        if (blk < nblk) {
          const int i0 = 64 * blk + mm;
          const float a = S[padx(i0)], b = S[padx(i0 + 16)], cc = S[padx(i0 + 32)], e = S[padx(i0 + 48)];
          S[padx(i0)] = a + b + cc - e;
          S[padx(i0 + 16)] = a + b - cc + e;
          S[padx(i0 + 32)] = a - b + cc + e;
          S[padx(i0 + 48)] = -a + b + cc + e;
        }
      }
  }
  row_sync<WPR>();
  // stride 64: quad w -> elements 256(w/64) + w%64 + 64k
  for (int w = tr; w < quads; w += T) {
    const int i0 = 256 * (w >> 6) + (w & 63);
    const float a = S[padx(i0)], b = S[padx(i0 + 64)], c = S[padx(i0 + 128)], e = S[padx(i0 + 192)];
    S[padx(i0)] = a + b + c - e;
    S[padx(i0 + 64)] = a + b - c + e;
    S[padx(i0 + 128)] = a - b + c + e;
    S[padx(i0 + 192)] = -a + b + c + e;
  }
  row_sync<WPR>();
}

// Row maximum of |v| over T threads (WPR waves share `red`).
template <int WPR>
__device__ __forceinline__ float row_max(float v, float* red, int tr) {
  v = wave_max(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    if ((tr & 63) == 0) red[tr >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < WPR; i++) r = fmaxf(r, red[i]);
    return r;
  }
}

// Rotated (x 1/16 if rotate) padded row -> optional fp32 Y, optional int8 q + per-row s
// (s = amax/127, q = clamp(rint(v * (127/amax)))).
template <int WPR>
__device__ __forceinline__ void quant_row_padded(const float* S, int cols, int tr, int rotate, float* red, float* Y,
                                                 int8_t* q, float* s_out) {
  constexpr int T = 64 * WPR;
  const int c4n = cols >> 2;
  float amax = 0.0f;
  for (int c4 = tr; c4 < c4n; c4 += T) {
    float4 v = *(const float4*)(S + padx(4 * c4));
    if (rotate) v = make_float4(v.x * 0.0625f, v.y * 0.0625f, v.z * 0.0625f, v.w * 0.0625f);
    if (Y) *(float4*)(Y + 4 * c4) = v;
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  if (!q) return;
  amax = row_max<WPR>(amax, red, tr);
  const float sc = amax / 127.0f, inv = 127.0f / amax;
  if (tr == 0) *s_out = sc;
  for (int c4 = tr; c4 < c4n; c4 += T) {
    float4 v = *(const float4*)(S + padx(4 * c4));
    if (rotate) v = make_float4(v.x * 0.0625f, v.y * 0.0625f, v.z * 0.0625f, v.w * 0.0625f);
    const float e[4] = {v.x, v.y, v.z, v.w};
    char4 o;
    int8_t* ob = (int8_t*)&o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float t = amax == 0.0f ? 0.0f : rintf(e[j] * inv);
      t = fminf(fmaxf(t, -127.0f), 127.0f);
      ob[j] = (int8_t)t;
    }
    *(char4*)(q + 4 * c4) = o;
  }
}

// Padded row floats of a row of `cols` (cols % 64 == 0 or the tail is unused padding-free).
__host__ __device__ constexpr int padded_cols(int cols) { return cols + 4 * ((cols + 63) / 64); }

// rows of K: optional rotation (K % 256 == 0), per-token int8.  WPR waves per row; a workgroup
// holds 4 / WPR rows; dynamic LDS = rows per workgroup * padded_cols(K) floats.
// activation of the preceding linear (ANIMA_ACT_*), applied to a loaded float4
__device__ __forceinline__ float act1(float v, int act) {
  return act == ANIMA_ACT_GELU ? gelu_erf(v) : act == ANIMA_ACT_SILU ? silu_f(v) : v;
}
__device__ __forceinline__ float4 act4(float4 v, int act) {
  return make_float4(act1(v.x, act), act1(v.y, act), act1(v.z, act), act1(v.w, act));
}

template <int WPR>
__global__ __launch_bounds__(256) void quant_rows_pad_kernel(const float* X, int64_t M, int K, int rotate, int act,
                                                             int8_t* Q, float* S_out) {
  extern __shared__ float SH[];
  __shared__ float red[4];
  constexpr int T = 64 * WPR;
  const int tr = threadIdx.x % T;
  const int64_t row = (int64_t)blockIdx.x * (4 / WPR) + threadIdx.x / T;
  if (row >= M) return;  // (a whole row's threads leave together; WPR > 1 launches one row per workgroup)
  float* S = SH + (size_t)(threadIdx.x / T) * padded_cols(K);
  const float* x = X + row * K;
  // every load of the row is issued before the first use (K <= 8 * 4 * T)
  float4 v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int c4 = tr + T * i;
    v[i] = c4 < (K >> 2) ? *(const float4*)(x + 4 * c4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  if (act != ANIMA_ACT_NONE) {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = act4(v[i], act);
  }
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int c4 = tr + T * i;
    if (c4 < (K >> 2)) *(float4*)(S + padx(4 * c4)) = rotate ? bfly4(v[i]) : v[i];
  }
  row_sync<WPR>();
  if (rotate) butterfly_stages234<WPR>(S, K, tr);
  quant_row_padded<WPR>(S, K, tr, rotate, red, nullptr, Q + row * K, S_out + row);
}

// ------------------------------------------------------------------ register-resident rows
//
// Rows of K = 1024, 2048, 4096 or 8192 columns: lane L of a row's LR = K/64 lanes holds the 64 consecutive
// elements 64L..64L+63, so a 256-element Hadamard block sits in 4 consecutive lanes (a DPP quad).
// Butterfly stages 1-3 (strides 1, 4, 16) combine elements of one lane; stage 4 (stride 64)
// combines the four lanes of the quad through DPP broadcasts.  Each stage applies the 4-point
// formula of the reference in its order: out_k = ((x0 s0 + x1 s1) + x2 s2) + x3 s3 with
// s_m = -1 exactly when m = 3 - k (kernels.js:359-388), so every fp32 result equals the LDS
// variant's.  No LDS except the cross-wave maximum of rows wider than a wave.

// 4-point butterfly of the reference on four values held by one lane (outputs in place)
// (-a + b is -(a - b) exactly, so the four outputs share a + b and a - b.)
__device__ __forceinline__ void bfly4_ref(float& a, float& b, float& c, float& e) {
  const float u = a + b, w = a - b;
  const float o0 = (u + c) - e, o1 = (u - c) + e, o2 = (w + c) + e, o3 = (c - w) + e;
  a = o0;
  b = o1;
  c = o2;
  e = o3;
}

// Hadamard (x 1/16 unless !SCALE) of the lane's 64 elements: stages 1-3 in registers, stage 4
// across the quad.
template <bool SCALE = true>
__device__ __forceinline__ void hadamard64_quad(float (&v)[64], int k) {
#pragma unroll
  for (int s = 1; s <= 16; s *= 4)
#pragma unroll
    for (int b = 0; b < 64; b++)
      if ((b / s) % 4 == 0) bfly4_ref(v[b], v[b + s], v[b + 2 * s], v[b + 3 * s]);
  const float s0 = k == 3 ? -1.0f : 1.0f, s1 = k == 2 ? -1.0f : 1.0f, s2 = k == 1 ? -1.0f : 1.0f,
              s3 = k == 0 ? -1.0f : 1.0f;
  // t = x0 s0, then t = fma(x_m, s_m, t) for m = 1..3, where x_m is v[p] of quad lane m: the DPP
  // forms of v_mul / v_fmac read x_m straight from lane m (one instruction per term instead of a
  // DPP move plus a VOP3 FMA).  s_nop 1: the two wait states gfx9 requires between a VALU write
  // of v[p] and a DPP read of it.
#pragma unroll
  for (int p = 0; p < 64; p++) {
    float t;
    asm volatile(
        "s_nop 1\n\t"
        "v_mul_f32_dpp %0, %1, %2 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %3 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %4 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %5 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf"
        : "=&v"(t)
        : "v"(v[p]), "v"(s0), "v"(s1), "v"(s2), "v"(s3));
    v[p] = SCALE ? t * 0.0625f : t;
  }
}

// Row maximum over the LR lanes of a row (LR <= 64: within the wave; 128: two waves via LDS).
template <int LR>
__device__ __forceinline__ float rows_max(float v, float* red) {
#pragma unroll
  for (int s = 1; s < (LR < 64 ? LR : 64); s *= 2) v = fmaxf(v, __shfl_xor(v, s));
  if constexpr (LR > 64) {
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    v = fmaxf(red[w & ~1], red[w | 1]);
  }
  return v;
}

// Per-token int8 of the lane's 64 values (q = clamp(rint(v * (127/amax))), s = amax/127).
// Rounding by the 1.5 * 2^23 add: for |r| < 2^22, r + C lies in [2^23, 2^24), where the float
// spacing is 1, so it equals C + rint(r) (ties to even; C is even) and its low byte is rint(r) in
// two's complement; the clamp to C -/+ 127 in float is the clamp to -/+127 (a NaN goes to -127
// as with fmaxf / fminf on the integer).
__device__ __forceinline__ void quant64_store(const float (&v)[64], float amax, int8_t* q) {
  // an all-zero row: inv = 0 gives q = 0, as the definition's special case
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  constexpr float C = 12582912.0f;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; d++) {
      uint32_t b[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float t = v[16 * g + 4 * d + j] * inv + C;
        b[j] = __float_as_uint(fminf(fmaxf(t, C - 127.0f), C + 127.0f));
      }
      // bytes 0 of b0, b1 (low half) and of b2, b3 (high half)
      w[d] = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u) | __builtin_amdgcn_perm(b[3], b[2], 0x04000c0cu);
    }
    *(uint4*)(q + 16 * g) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// rows of K = 64 * LR columns (LR = 16, 32, 64, 128), optional activation and Hadamard, per-token int8.
// 256 threads: 256 / LR rows per workgroup (LR = 128: one row over two waves, two per workgroup).
template <int LR>
__global__ __launch_bounds__(256) void quant_rows_reg_kernel(const float* X, int64_t M, int rotate, int act, int8_t* Q,
                                                             float* S_out) {
  constexpr int K = 64 * LR;
  __shared__ float red[4];
  const int L = threadIdx.x % LR;
  const int64_t row = (int64_t)blockIdx.x * (256 / LR) + threadIdx.x / LR;
  const bool live = row < M;  // (dead rows still take part in the cross-wave maximum)
  const float* x = X + (live ? row : 0) * K + 64 * L;
  float v[64];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const float4 t = *(const float4*)(x + 4 * i);
    v[4 * i] = t.x;
    v[4 * i + 1] = t.y;
    v[4 * i + 2] = t.z;
    v[4 * i + 3] = t.w;
  }
  if (act != ANIMA_ACT_NONE) {
#pragma unroll
    for (int i = 0; i < 64; i++) v[i] = act1(v[i], act);
  }
  // The Hadamard's final 1/16 is left out: scaling a row by a power of two scales its maximum
  // the same way and leaves q = rint(v * (127 / amax)) unchanged (127 / (amax / 16) is exactly
  // 16 * (127 / amax) and the products are equal), so only the stored scale takes it.
  if (rotate) hadamard64_quad<false>(v, L & 3);
  float am = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; i++) am = fmaxf(am, fabsf(v[i]));
  am = rows_max<LR>(am, red);
  if (!live) return;
  if (L == 0) S_out[row] = (rotate ? am * 0.0625f : am) / 127.0f;
  quant64_store(v, am, Q + row * K + 64 * L);
}

// quant_rows_reg_kernel on bf16 rows: each lane's 64 values arrive as eight 16-byte loads of
// bf16 and are widened exactly (bits << 16), then the same Hadamard, maximum and int8 rounding.
template <int LR>
__global__ __launch_bounds__(256) void quant_rows_bf16_kernel(const uint16_t* X, int64_t M, int rotate, int8_t* Q,
                                                              float* S_out) {
  constexpr int K = 64 * LR;
  __shared__ float red[4];
  const int L = threadIdx.x % LR;
  const int64_t row = (int64_t)blockIdx.x * (256 / LR) + threadIdx.x / LR;
  const bool live = row < M;  // (dead rows still take part in the cross-wave maximum)
  const uint16_t* x = X + (live ? row : 0) * K + 64 * L;
  float v[64];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint4 t = *(const uint4*)(x + 8 * i);
    const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[8 * i + 2 * e] = __uint_as_float(w[e] << 16);
      v[8 * i + 2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  }
  if (rotate) hadamard64_quad<false>(v, L & 3);
  float am = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; i++) am = fmaxf(am, fabsf(v[i]));
  am = rows_max<LR>(am, red);
  if (!live) return;
  if (L == 0) S_out[row] = (rotate ? am * 0.0625f : am) / 127.0f;
  quant64_store(v, am, Q + row * K + 64 * L);
}

// LayerNorm (no affine) + adaLN (+ Hadamard) (+ int8), one wave per row (app/gpu/kernels.js:108-145).
// Lane l holds the float4 chunks l, l+64, ... i.e. elements 4l + j + 256i, exactly the elements
// the reference's 256-thread loops give to threads 4l + j, so the strided partial sums and the
// 128..1 tree ("red[t] += red[t + s]") are reproduced term for term (wave_tree_sum4).
__device__ __forceinline__ float wave_tree_sum4(float p0, float p1, float p2, float p3) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    const float q0 = __shfl_down(p0, s), q1 = __shfl_down(p1, s), q2 = __shfl_down(p2, s), q3 = __shfl_down(p3, s);
    p0 = p0 + q0;
    p1 = p1 + q1;
    p2 = p2 + q2;
    p3 = p3 + q3;
  }
  p0 = p0 + p2;
  p1 = p1 + p3;
  return __shfl(p0 + p1, 0);
}

__global__ __launch_bounds__(256) void layernorm_mod_wave_kernel(const float* X, const float* MOD, int64_t shift_off,
                                                                 int64_t scale_off, int64_t rows, int cols, float eps,
                                                                 int rotate, float* Y, int8_t* Q, float* S_out) {
  extern __shared__ float SH[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= rows) return;
  float* S = SH + (size_t)wave * padded_cols(cols);
  const float* x = X + row * cols;
  const int c4n = cols >> 2;
  // the row stays in registers (every load issued before the first use; cols <= 2048);
  // per-thread partial sums of the virtual threads 4*lane + j
  float4 xv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int c4 = lane + 64 * i;
    xv[i] = c4 < c4n ? *(const float4*)(x + 4 * c4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int c4 = lane + 64 * i;
    if (c4 < c4n) {
      const float4 v = xv[i];
      p0 += v.x;
      p1 += v.y;
      p2 += v.z;
      p3 += v.w;
    }
  }
  const float mean = wave_tree_sum4(p0, p1, p2, p3) / (float)cols;
  p0 = p1 = p2 = p3 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    if (lane + 64 * i >= c4n) break;
    const float4 v = xv[i];
    const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
    p0 += d0 * d0;
    p1 += d1 * d1;
    p2 += d2 * d2;
    p3 += d3 * d3;
  }
  const float r = 1.0f / sqrtf(wave_tree_sum4(p0, p1, p2, p3) / (float)cols + eps);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int c4 = lane + 64 * i;
    if (c4 >= c4n) break;
    const float4 v = xv[i];
    const float4 sc = *(const float4*)(MOD + scale_off + 4 * c4);
    const float4 sh = *(const float4*)(MOD + shift_off + 4 * c4);
    const float4 n = make_float4((v.x - mean) * r * (1.0f + sc.x) + sh.x, (v.y - mean) * r * (1.0f + sc.y) + sh.y,
                                 (v.z - mean) * r * (1.0f + sc.z) + sh.z, (v.w - mean) * r * (1.0f + sc.w) + sh.w);
    *(float4*)(S + padx(4 * c4)) = rotate ? bfly4(n) : n;
  }
  if (rotate) butterfly_stages234<1>(S, cols, lane);
  quant_row_padded<1>(S, cols, lane, rotate, nullptr, Y ? Y + row * cols : nullptr, Q ? Q + row * cols : nullptr,
                      Q ? S_out + row : nullptr);
}

// LayerNorm + adaLN (+ Hadamard) (+ int8) for rows of 64 LR columns (LR = 16, 32), LR lanes per
// row, 256 / LR rows per workgroup, no workgroup barrier.  Statistics: lane l holds the VT = 256 / LR
// consecutive elements VT l + j of every 256-column block, i.e. exactly the elements the
// reference's 256-thread loops give to threads VT l + j (kernels.js:108-145), so the strided
// partial sums and the "red[t] += red[t + s]" tree are reproduced term for term (the partner of
// t = VT l + j at level s >= VT is lane l + s / VT, below VT it is in-lane).  The modulated row then
// crosses LDS once (padded by 4 floats per 64: conflict-free 16-byte writes and reads) into the
// register-Hadamard layout (lane l holds 64 l .. 64 l + 63) and leaves as int8 and / or fp32.
template <int LR>
__device__ __forceinline__ float seg_tree_sum(float (&p)[256 / LR]) {
  constexpr int VT = 256 / LR;
#pragma unroll
  for (int s = 128; s >= 1; s >>= 1) {
    if (s >= VT) {
#pragma unroll
      for (int j = 0; j < VT; j++) {
        const float q = __shfl_down(p[j], s / VT, LR);
        p[j] = p[j] + q;
      }
    } else {
#pragma unroll
      for (int j = 0; j < s; j++) p[j] = p[j] + p[j + s];
    }
  }
  return __shfl(p[0], 0, LR);
}

template <int LR>
__global__ __launch_bounds__(256) void layernorm_mod_reg_kernel(const float* X, const float* MOD, int64_t shift_off,
                                                                int64_t scale_off, int64_t rows, float eps, int rotate,
                                                                float* Y, int8_t* Q, float* S_out) {
  // The modulated row crosses LDS in two halves of COLS / 2 columns through one half-row buffer:
  // 34-38 KiB per workgroup instead of 68-76, so four workgroups (four waves per SIMD) fit on a CU
  // instead of two.  A 16-byte LDS access is served eight lanes at a time over 32 banks, so the
  // 16-byte slots of any eight consecutive lanes must differ modulo 8.  LR = 32: the writers
  // (lane x, slot 2x + q of a 256-column block) and the readers (lane lh, slots 16 lh + q') both
  // meet that with 4 floats of padding after every 32 columns and 4 more after every 64 (slot n
  // at n + n/8 + n/16); LR = 16 keeps 4 floats per 64.
  constexpr int COLS = 64 * LR, VT = 256 / LR, NB = COLS / 256, RPW = 256 / LR, HB = NB / 2;
  constexpr int RS = LR == 32 ? COLS / 2 + COLS / 16 + COLS / 32 : COLS / 2 + 2 * LR;  // half-row stride in floats
  __shared__ __attribute__((aligned(16))) float SH[RPW * RS];
  const int l = threadIdx.x % LR, rl = threadIdx.x / LR;
  const int64_t row = (int64_t)blockIdx.x * RPW + rl;
  if (row >= rows) return;  // (a row's lanes leave together; nothing below spans rows)
  const float* x = X + row * COLS + VT * l;
  // padded LDS offsets of this lane's writes (column 256 i' + VT l + 4 q of the half: wb + the
  // compile-time 304 i' + 4 q for LR = 32, whose q < 2) and reads (columns 64 lh + 4 q)
  const int wb = LR == 32 ? 8 * l + 4 * (l >> 2) + 4 * (l >> 3) : VT * l + 4 * ((VT * l) >> 6);
  float v[64];  // v[VT i + j] = x[256 i + VT l + j]
#pragma unroll
  for (int i = 0; i < NB; i++)
#pragma unroll
    for (int q = 0; q < VT / 4; q++) {
      const float4 t = *(const float4*)(x + 256 * i + 4 * q);
      v[VT * i + 4 * q] = t.x;
      v[VT * i + 4 * q + 1] = t.y;
      v[VT * i + 4 * q + 2] = t.z;
      v[VT * i + 4 * q + 3] = t.w;
    }
  float p[VT];
#pragma unroll
  for (int j = 0; j < VT; j++) p[j] = 0.0f;
#pragma unroll
  for (int i = 0; i < NB; i++)
#pragma unroll
    for (int j = 0; j < VT; j++) p[j] += v[VT * i + j];
  const float mean = seg_tree_sum<LR>(p) / (float)COLS;
#pragma unroll
  for (int j = 0; j < VT; j++) p[j] = 0.0f;
#pragma unroll
  for (int i = 0; i < NB; i++)
#pragma unroll
    for (int j = 0; j < VT; j++) {
      const float d = v[VT * i + j] - mean;
      p[j] += d * d;
    }
  const float r = 1.0f / sqrtf(seg_tree_sum<LR>(p) / (float)COLS + eps);
  float* S = SH + rl * RS;
  // Half hh: every lane writes its elements of columns [hh * COLS / 2, (hh + 1) * COLS / 2)
  // (blocks hh * HB .. + HB), then the LR / 2 lanes whose 64 Hadamard columns lie in that half
  // read them.  The row's lanes all belong to this wave and LDS operations of one wave complete
  // in order; the wavefront-scope fences keep the compiler from moving a half's reads above its
  // writes, or the second half's writes above the first half's reads.
  float w[64];
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
#pragma unroll
    for (int i = hh * HB; i < (hh + 1) * HB; i++)
#pragma unroll
      for (int q = 0; q < VT / 4; q++) {
        const int c = 256 * i + VT * l + 4 * q, ih = i - hh * HB;
        const float4 sc = *(const float4*)(MOD + scale_off + c);
        const float4 sh = *(const float4*)(MOD + shift_off + c);
        const float* t = v + VT * i + 4 * q;
        *(float4*)(S + wb + (LR == 32 ? 304 * ih : (256 + 16) * ih) + 4 * q) =
            make_float4((t[0] - mean) * r * (1.0f + sc.x) + sh.x, (t[1] - mean) * r * (1.0f + sc.y) + sh.y,
                        (t[2] - mean) * r * (1.0f + sc.z) + sh.z, (t[3] - mean) * r * (1.0f + sc.w) + sh.w);
      }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (l / (LR / 2) == hh) {
      const int lh = l - hh * (LR / 2);
#pragma unroll
      for (int q = 0; q < 16; q++) {
        const float4 t = *(const float4*)(S + (LR == 32 ? 76 * lh + 4 * q + 4 * (q >> 3) : 68 * lh + 4 * q));
        w[4 * q] = t.x;
        w[4 * q + 1] = t.y;
        w[4 * q + 2] = t.z;
        w[4 * q + 3] = t.w;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  }
  if (rotate) hadamard64_quad(w, l & 3);
  if (Y) {
    float* y = Y + row * COLS + 64 * l;
#pragma unroll
    for (int q = 0; q < 16; q++) *(float4*)(y + 4 * q) = make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
  }
  if (Q) {
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; i++) am = fmaxf(am, fabsf(w[i]));
    am = rows_max<LR>(am, nullptr);
    if (l == 0) S_out[row] = am / 127.0f;
    quant64_store(w, am, Q + row * COLS + 64 * l);
  }
}

__global__ __launch_bounds__(256) void elementwise_kernel(int op, const float* A, const float* B, float* Y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float a = A ? A[i] : 0.0f;
    float y;
    switch (op) {
      case ANIMA_EW_SILU_MUL: y = silu_f(a) * B[i]; break;
      case ANIMA_EW_ADD: y = a + B[i]; break;
      case ANIMA_EW_SILU: y = silu_f(a); break;
      default: y = a; break;
    }
    Y[i] = y;
  }
}

// 16-byte copy / fill (elementwise copy on aligned buffers, zero).
__global__ __launch_bounds__(256) void copy4_kernel(const float4* A, float4* Y, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256)
    Y[i] = A ? A[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// Grid of the grid-stride element kernels: at most 1024 workgroups (4 per CU), where a 16-byte
// copy moved the most bytes per second (fewer, longer-lived waves than one per 256 elements).
static unsigned grid_for(int64_t n) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 1024)); }

int hadamard_launch(anima_ctx* c, const float* x, float* y, int64_t n) {
  if (!x || !y) return fail(c, ANIMA_E_ARG, "anima_hadamard: null pointer");
  if (n < 0 || n % 256) return fail(c, ANIMA_E_ARG, "anima_hadamard: n=%lld must be a multiple of 256", (long long)n);
  if (n == 0) return ANIMA_OK;
  const int64_t groups = n / 256;
  Launch lc(c, "hadamard", 0.0, (double)n * 8);
  hipLaunchKernelGGL(hadamard_kernel, dim3((unsigned)((groups + 3) / 4)), dim3(256), 0, c->stream, x, y, groups);
  return lc.end();
}

int quant_rows_launch(anima_ctx* c, const float* x, int64_t M, int K, int rotate, int act, int8_t* q, float* s) {
  if (!x || !q || !s) return fail(c, ANIMA_E_ARG, "anima_quant_rows: null pointer");
  if (act < ANIMA_ACT_NONE || act > ANIMA_ACT_SILU) return fail(c, ANIMA_E_ARG, "anima_quant_rows_act: unknown act %d", act);
  if (M < 0 || K < 4 || K % 4 || K > 8192 || (rotate && K % 256))
    return fail(c, ANIMA_E_ARG, "anima_quant_rows: M=%lld K=%d (K %% 4 == 0, <= 8192, %% 256 == 0 when rotating)", (long long)M, K);
  if (M > 0x7fffffff) return fail(c, ANIMA_E_ARG, "anima_quant_rows: M too large");
  if (((uintptr_t)x & 15) || ((uintptr_t)q & 3)) return fail(c, ANIMA_E_ARG, "anima_quant_rows: x must be 16-byte and q 4-byte aligned");
  if (M == 0) return ANIMA_OK;
  Launch lc(c, act ? "act_hadamard_quant" : rotate ? "hadamard_quant" : "quant_rows", 0.0, (double)M * K * 5 + M * 4.0);
  // register-resident rows for the widths with a kernel instance (a row of K = 64 LR columns)
  if ((K == 1024 || K == 2048 || K == 4096 || K == 8192) && !((uintptr_t)q & 15)) {
    const unsigned rows_per = 256 / (K / 64);
    const dim3 grid((unsigned)((M + rows_per - 1) / rows_per));
    switch (K) {
      case 1024: hipLaunchKernelGGL(quant_rows_reg_kernel<16>, grid, dim3(256), 0, c->stream, x, M, rotate, act, q, s); break;
      case 2048: hipLaunchKernelGGL(quant_rows_reg_kernel<32>, grid, dim3(256), 0, c->stream, x, M, rotate, act, q, s); break;
      case 4096: hipLaunchKernelGGL(quant_rows_reg_kernel<64>, grid, dim3(256), 0, c->stream, x, M, rotate, act, q, s); break;
      case 8192: hipLaunchKernelGGL(quant_rows_reg_kernel<128>, grid, dim3(256), 0, c->stream, x, M, rotate, act, q, s); break;
    }
    return lc.end();
  }
  if (K > 2048)  // four waves per row, one row per workgroup (at most 35 KB of LDS)
    hipLaunchKernelGGL(quant_rows_pad_kernel<4>, dim3((unsigned)M), dim3(256), (size_t)padded_cols(K) * 4, c->stream, x, M,
                       K, rotate, act, q, s);
  else  // one wave per row, four rows per workgroup
    hipLaunchKernelGGL(quant_rows_pad_kernel<1>, dim3((unsigned)((M + 3) / 4)), dim3(256), (size_t)4 * padded_cols(K) * 4,
                       c->stream, x, M, K, rotate, act, q, s);
  return lc.end();
}

int quant_rows_bf16_launch(anima_ctx* c, const uint16_t* x, int64_t M, int K, int rotate, int8_t* q, float* s) {
  if (!x || !q || !s) return fail(c, ANIMA_E_ARG, "anima_quant_rows_bf16: null pointer");
  if (M < 0 || M > 0x7fffffff || (K != 1024 && K != 2048 && K != 4096 && K != 8192))
    return fail(c, ANIMA_E_ARG, "anima_quant_rows_bf16: M=%lld K=%d (K = 1024, 2048, 4096 or 8192)", (long long)M, K);
  if (((uintptr_t)x & 15) || ((uintptr_t)q & 15)) return fail(c, ANIMA_E_ARG, "anima_quant_rows_bf16: x and q must be 16-byte aligned");
  if (M == 0) return ANIMA_OK;
  Launch lc(c, rotate ? "hadamard_quant_bf16" : "quant_rows_bf16", 0.0, (double)M * K * 3 + M * 4.0);
  const dim3 grid((unsigned)((M + 256 / (K / 64) - 1) / (256 / (K / 64))));
  switch (K) {
    case 1024: hipLaunchKernelGGL(quant_rows_bf16_kernel<16>, grid, dim3(256), 0, c->stream, x, M, rotate, q, s); break;
    case 2048: hipLaunchKernelGGL(quant_rows_bf16_kernel<32>, grid, dim3(256), 0, c->stream, x, M, rotate, q, s); break;
    case 4096: hipLaunchKernelGGL(quant_rows_bf16_kernel<64>, grid, dim3(256), 0, c->stream, x, M, rotate, q, s); break;
    default: hipLaunchKernelGGL(quant_rows_bf16_kernel<128>, grid, dim3(256), 0, c->stream, x, M, rotate, q, s); break;
  }
  return lc.end();
}

int layernorm_mod_launch(anima_ctx* c, const float* x, const float* mod, int64_t shift_off, int64_t scale_off,
                         int64_t rows, int cols, float eps, int rotate, float* y, int8_t* q, float* s) {
  if (!x || !mod) return fail(c, ANIMA_E_ARG, "anima_layernorm_mod: null x or mod");
  if (!y && !q) return fail(c, ANIMA_E_ARG, "anima_layernorm_mod: no output (y or q)");
  if (q && (!s || !rotate)) return fail(c, ANIMA_E_ARG, "anima_layernorm_mod: int8 output needs s and rotate");
  if (rows < 0 || rows > 0x7fffffff || cols < 4 || cols % 4 || cols > 8192 || (rotate && cols % 256))
    return fail(c, ANIMA_E_ARG, "anima_layernorm_mod: rows=%lld cols=%d", (long long)rows, cols);
  if (shift_off < 0 || scale_off < 0) return fail(c, ANIMA_E_ARG, "anima_layernorm_mod: negative offsets");
  if (q && ((uintptr_t)q & 3)) return fail(c, ANIMA_E_ARG, "anima_layernorm_mod: q must be 4-byte aligned");
  if (rows == 0) return ANIMA_OK;
  const double bytes = (double)rows * cols * 4 + (y ? rows * (double)cols * 4 : 0) + (q ? rows * (double)cols + rows * 4.0 : 0);
  Launch lc(c, q ? "layernorm_mod_rot_quant" : (rotate ? "layernorm_mod_rot" : "layernorm_mod"), 0.0, bytes);
  const bool vec = cols <= 2048 && !((uintptr_t)x & 15) && !((uintptr_t)(mod + shift_off) & 15) &&
                   !((uintptr_t)(mod + scale_off) & 15) && !((uintptr_t)y & 15);
  if (vec && (cols == 1024 || cols == 2048) && !((uintptr_t)q & 15)) {  // register rows, one LDS round trip
    if (cols == 2048)
      hipLaunchKernelGGL(layernorm_mod_reg_kernel<32>, dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, c->stream, x, mod,
                         shift_off, scale_off, rows, eps, rotate, y, q, s);
    else
      hipLaunchKernelGGL(layernorm_mod_reg_kernel<16>, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, c->stream, x, mod,
                         shift_off, scale_off, rows, eps, rotate, y, q, s);
  } else if (vec) {  // float4 rows: one wave per row
    hipLaunchKernelGGL(layernorm_mod_wave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256),
                       (size_t)4 * padded_cols(cols) * 4, c->stream, x, mod, shift_off, scale_off, rows, cols, eps, rotate, y,
                       q, s);
  } else {
    hipLaunchKernelGGL(layernorm_mod_kernel, dim3((unsigned)rows), dim3(256), (size_t)cols * 4, c->stream, x, mod, shift_off,
                       scale_off, cols, eps, rotate, y, q, s);
  }
  return lc.end();
}

int elementwise_launch(anima_ctx* c, int op, const float* a, const float* b, float* y, int64_t n) {
  if (op < ANIMA_EW_SILU_MUL || op > ANIMA_EW_COPY) return fail(c, ANIMA_E_ARG, "anima_elementwise: unknown op %d", op);
  if (!a || !y || ((op == ANIMA_EW_SILU_MUL || op == ANIMA_EW_ADD) && !b)) return fail(c, ANIMA_E_ARG, "anima_elementwise: null pointer");
  if (n < 0) return fail(c, ANIMA_E_ARG, "anima_elementwise: n < 0");
  if (n == 0) return ANIMA_OK;
  static const char* names[] = {"elementwise.silu_mul", "elementwise.add", "elementwise.silu", "elementwise.copy"};
  const int nin = (op == ANIMA_EW_SILU_MUL || op == ANIMA_EW_ADD) ? 2 : 1;
  Launch lc(c, names[op], 0.0, (double)n * 4 * (nin + 1));
  if (op == ANIMA_EW_COPY && n % 4 == 0 && !((uintptr_t)a & 15) && !((uintptr_t)y & 15))
    hipLaunchKernelGGL(copy4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, c->stream, (const float4*)a, (float4*)y, n / 4);
  else
    hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(n)), dim3(256), 0, c->stream, op, a, b, y, n);
  return lc.end();
}

int zero_launch(anima_ctx* c, float* y, int64_t n) {
  if (!y || n < 0) return fail(c, ANIMA_E_ARG, "anima_zero: bad arguments");
  if (n == 0) return ANIMA_OK;
  Launch lc(c, "zero", 0.0, (double)n * 4);
  if (n % 4 == 0 && !((uintptr_t)y & 15))
    hipLaunchKernelGGL(copy4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, c->stream, (const float4*)nullptr, (float4*)y, n / 4);
  else
    hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(n)), dim3(256), 0, c->stream, (int)ANIMA_EW_COPY, (const float*)nullptr,
                       (const float*)nullptr, y, n);
  return lc.end();
}

// Patch layout of the DiT input/output (app/models/dit.js:55-78).  Forward: one thread per patch
// element, [B*Hp*Wp][68] <- latents [B][16][h][w] (columns 64..67 zero).  Inverse: one thread per
// latent element, latents <- [B*Hp*Wp][64] in (p1 p2 c) order.
__global__ __launch_bounds__(256) void patchify_kernel(const float* lat, float* P, int h, int w, int64_t n) {
  const int Wp = w / 2, L = (h / 2) * Wp;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / 68;
    const int k = (int)(i - row * 68);
    const int64_t b = row / L;
    const int p = (int)(row - b * L), y = p / Wp, x = p - y * Wp;
    float v = 0.0f;
    if (k < 64) {
      const int c = k >> 2, m = (k >> 1) & 1, nn = k & 1;
      v = lat[((b * 16 + c) * h + 2 * y + m) * (int64_t)w + 2 * x + nn];
    }
    P[i] = v;
  }
}

__global__ __launch_bounds__(256) void unpatchify_kernel(const float* O, float* lat, int h, int w, int64_t n) {
  const int Wp = w / 2, L = (h / 2) * Wp;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t bc = i / ((int64_t)h * w);
    const int r = (int)(i - bc * h * w), yy = r / w, xx = r - yy * w;
    const int64_t b = bc / 16;
    const int c = (int)(bc - b * 16);
    const int64_t row = b * L + (yy >> 1) * Wp + (xx >> 1);
    lat[i] = O[row * 64 + (yy & 1) * 32 + (xx & 1) * 16 + c];
  }
}

int patchify_launch(anima_ctx* c, const float* src, float* dst, int B, int h, int w, bool inverse) {
  const char* fn = inverse ? "anima_unpatchify" : "anima_patchify";
  if (!src || !dst) return fail(c, ANIMA_E_ARG, "%s: null pointer", fn);
  if (B <= 0 || h <= 0 || w <= 0 || (h & 1) || (w & 1))
    return fail(c, ANIMA_E_ARG, "%s: B=%d h=%d w=%d (positive, h and w even)", fn, B, h, w);
  const int64_t nl = (int64_t)B * 16 * h * w, np = (int64_t)B * (h / 2) * (w / 2);
  if (!inverse) {
    Launch lc(c, "patchify", 0.0, (double)nl * 4 + (double)np * 68 * 4);
    hipLaunchKernelGGL(patchify_kernel, dim3(grid_for(np * 68)), dim3(256), 0, c->stream, src, dst, h, w, np * 68);
    return lc.end();
  }
  Launch lc(c, "unpatchify", 0.0, (double)nl * 8);
  hipLaunchKernelGGL(unpatchify_kernel, dim3(grid_for(nl)), dim3(256), 0, c->stream, src, dst, h, w, nl);
  return lc.end();
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_kernel(void* dst, int64_t n, int kind, uint64_t seed, float lo, float hi,
                                                   int64_t imul) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const uint64_t h = splitmix64(seed * 0xD1B54A32D192ED03ull + (uint64_t)i);
    switch (kind) {
      case ANIMA_FILL_U8: {
        const int64_t a = (int64_t)lo, b = (int64_t)hi;
        ((uint8_t*)dst)[i] = (uint8_t)(a + (int64_t)(h % (uint64_t)(b - a + 1)));
        break;
      }
      case ANIMA_FILL_I8N: {
        const int64_t sum = (int64_t)(h & 0xff) + (int64_t)((h >> 8) & 0xff) + (int64_t)((h >> 16) & 0xff) +
                            (int64_t)((h >> 24) & 0xff);
        int64_t v = ((sum - 510) * imul) >> 12;
        v = v < -127 ? -127 : (v > 127 ? 127 : v);
        ((int8_t*)dst)[i] = (int8_t)v;
        break;
      }
      case ANIMA_FILL_F32N: {
        const float u = (float)(h & 0xffff) * (1.0f / 65536.0f) + (float)((h >> 16) & 0xffff) * (1.0f / 65536.0f) +
                        (float)((h >> 32) & 0xffff) * (1.0f / 65536.0f) + (float)((h >> 48) & 0xffff) * (1.0f / 65536.0f);
        ((float*)dst)[i] = (u - 2.0f) * 1.7320508f * lo + hi;
        break;
      }
      default: {
        const float u = (float)(h >> 40) * (1.0f / 16777216.0f);
        const float v = lo + (hi - lo) * u;
        if (kind == ANIMA_FILL_F32) ((float*)dst)[i] = v;
        else ((bf16*)dst)[i] = to_bf16(v);
        break;
      }
    }
  }
}

int fill_random_launch(anima_ctx* c, void* dst, int64_t n, int kind, uint64_t seed, float lo, float hi) {
  if (!dst || n < 0) return fail(c, ANIMA_E_ARG, "anima_fill_random: bad arguments");
  if (kind < ANIMA_FILL_U8 || kind > ANIMA_FILL_F32N) return fail(c, ANIMA_E_ARG, "anima_fill_random: unknown kind %d", kind);
  if (kind == ANIMA_FILL_U8 && !(lo >= 0 && hi <= 255 && lo <= hi)) return fail(c, ANIMA_E_ARG, "anima_fill_random: u8 range [%g,%g]", lo, hi);
  if (n == 0) return ANIMA_OK;
  const int64_t imul = (int64_t)llrint((double)lo * 4096.0 / 147.8017);
  Launch lc(c, "fill_random", 0.0, (double)n);
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n)), dim3(256), 0, c->stream, dst, n, kind, seed, lo, hi, imul);
  return lc.end();
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
