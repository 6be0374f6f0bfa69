/*
 * CPU oracle for the DiT attention hot path -- TEST INFRASTRUCTURE ONLY.
 * Restates the reference's arithmetic in plain C (compiled with -ffp-contract=off so every
 * fp32 operation rounds where the reference's source rounds).  Only tests/, the smoke check
 * and the bench's CPU-baseline leg use it; the product never links it.
 * Citations are relative to the anima-studio repository.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ RNG (app/rng.js:5-67) */

typedef struct {
  uint32_t mt[624];
  int idx;
} mt19937;

static void mt_seed(mt19937* g, uint32_t seed) { /* app/rng.js:6-14 */
  g->mt[0] = seed;
  for (int i = 1; i < 624; i++) {
    uint32_t p = g->mt[i - 1] ^ (g->mt[i - 1] >> 30);
    g->mt[i] = 1812433253u * p + (uint32_t)i;
  }
  g->idx = 624;
}

static void mt_twist(mt19937* g) { /* app/rng.js:15-24 */
  for (int i = 0; i < 624; i++) {
    uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
    uint32_t v = g->mt[(i + 397) % 624] ^ (y >> 1);
    if (y & 1u) v ^= 0x9908b0dfu;
    g->mt[i] = v;
  }
  g->idx = 0;
}

static uint32_t mt_next(mt19937* g) { /* app/rng.js:25-33 */
  if (g->idx >= 624) mt_twist(g);
  uint32_t y = g->mt[g->idx++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

void orc_mt19937(uint32_t seed, int64_t n, uint32_t* out) {
  mt19937 g;
  mt_seed(&g, seed);
  for (int64_t i = 0; i < n; i++) out[i] = mt_next(&g);
}

static float uniform24(mt19937* g) { /* app/rng.js:41-43: 24 random bits */
  return (float)((double)(mt_next(g) & 0xffffffu) / 16777216.0);
}

static void fill16(float* d) { /* app/rng.js:44-53 (Box-Muller on 8 pairs) */
  for (int j = 0; j < 8; j++) {
    float u1 = 1.0f - d[j];
    float u2 = d[j + 8];
    float lg = (float)log((double)u1);
    float radius = (float)sqrt((double)(float)(-2.0 * (double)lg));
    float theta = (float)(2.0 * 3.14159265358979323846 * (double)u2);
    d[j] = radius * (float)cos((double)theta);
    d[j + 8] = radius * (float)sin((double)theta);
  }
}

void orc_randn(uint64_t seed, int64_t n, float* d) { /* app/rng.js:55-66 */
  mt19937 g;
  mt_seed(&g, (uint32_t)seed);
  if (n < 16) return;
  for (int64_t i = 0; i < n; i++) d[i] = uniform24(&g);
  for (int64_t i = 0; i + 16 <= n; i += 16) fill16(d + i);
  if (n % 16 != 0) {
    float* o = d + (n - 16);
    for (int i = 0; i < 16; i++) o[i] = uniform24(&g);
    fill16(o);
  }
}

/* ------------------------------------------------------------------ RoPE tables */

void orc_dit_rope_angles(int Hp, int Wp, float* a) { /* app/models/common.js:31-52 */
  const int head_dim = 128;
  const int dim_h = (head_dim / 6) * 2; /* 42 */
  const int dim_t = head_dim - 2 * dim_h; /* 44 */
  const double h_theta = 10000.0 * pow(4.0, (double)dim_h / (double)(dim_h - 2));
  float hf[21];
  for (int j = 0; j < dim_h / 2; j++) {
    float ex = (float)((double)(2 * j) / (double)dim_h);
    hf[j] = (float)(1.0 / pow(h_theta, (double)ex));
  }
  const int half = 64;
  memset(a, 0, sizeof(float) * (size_t)Hp * Wp * half);
  for (int y = 0; y < Hp; y++)
    for (int x = 0; x < Wp; x++) {
      float* o = a + ((size_t)y * Wp + x) * half;
      for (int j = 0; j < 21; j++) {
        o[dim_t / 2 + j] = (float)((double)y * (double)hf[j]);
        o[dim_t / 2 + 21 + j] = (float)((double)x * (double)hf[j]);
      }
    }
}

void orc_rope_table(const float* ang, int64_t L, int half, float* cs) { /* common.js:3-12 */
  for (int64_t i = 0; i < L * half; i++) {
    cs[i] = (float)cos((double)ang[i]);
    cs[L * half + i] = (float)sin((double)ang[i]);
  }
}

/* ------------------------------------------------------------------ row kernels */

/* Tree reduction of red[0..n) with the shader's stride order (s = n/2 ... 1). */
static float tree_sum(float* red, int n) {
  for (int s = n / 2; s > 0; s >>= 1)
    for (int i = 0; i < s; i++) red[i] = red[i] + red[i + s];
  return red[0];
}

void orc_qk_norm_rope(float* X, int64_t L, int H, int D, int64_t ld, const float* QN,
                      const float* KN, const float* CS, int64_t sin_off, float eps) {
  /* app/gpu/kernels.js:314-333: one workgroup of D/2 threads per (token, q-or-k head) */
  const int half = D / 2;
  float red[256];
  for (int64_t l = 0; l < L; l++)
    for (int h = 0; h < 2 * H; h++) {
      float* base = X + l * ld + (int64_t)h * D;
      for (int i = 0; i < half; i++) red[i] = base[i] * base[i] + base[i + half] * base[i + half];
      float r = 1.0f / sqrtf(tree_sum(red, half) / (float)D + eps);
      const float* w = h < H ? QN : KN;
      for (int i = 0; i < half; i++) {
        float x1 = base[i], x2 = base[i + half];
        float y1 = x1 * r * w[i];
        float y2 = x2 * r * w[i + half];
        float c = CS[l * half + i];
        float s = CS[sin_off + l * half + i];
        base[i] = y1 * c - y2 * s;
        base[i + half] = y2 * c + y1 * s;
      }
    }
}

void orc_rmsnorm(const float* X, const float* W, float* Y, int64_t rows, int cols, float eps) {
  /* app/gpu/kernels.js:73-88: 64 threads stride the row, then a 32..1 tree */
  float red[64];
  for (int64_t row = 0; row < rows; row++) {
    const float* x = X + row * cols;
    for (int t = 0; t < 64; t++) {
      float ss = 0.0f;
      for (int c = t; c < cols; c += 64) ss += x[c] * x[c];
      red[t] = ss;
    }
    float r = 1.0f / sqrtf(tree_sum(red, 64) / (float)cols + eps);
    for (int c = 0; c < cols; c++) Y[row * cols + c] = x[c] * r * W[c];
  }
}

void orc_rope(float* X, const float* CS, int64_t L, int H, int D, int64_t sin_off,
              int64_t row_stride, int64_t col_off) { /* app/gpu/kernels.js:343-356 */
  const int half = D / 2;
  for (int64_t l = 0; l < L; l++)
    for (int h = 0; h < H; h++)
      for (int i = 0; i < half; i++) {
        float* base = X + l * row_stride + col_off + (int64_t)h * D;
        float c = CS[l * half + i], s = CS[sin_off + l * half + i];
        float x1 = base[i], x2 = base[i + half];
        base[i] = x1 * c - x2 * s;
        base[i + half] = x2 * c + x1 * s;
      }
}

/* One 256-group butterfly pass set, in place (app/gpu/kernels.js:373-386 and 124-140). */
static void butterfly256(float* s) {
  int stride = 1;
  for (int d = 0; d < 4; d++) {
    for (int t = 0; t < 64; t++) {
      int lo = t % stride;
      int i0 = (t / stride) * stride * 4 + lo;
      float a = s[i0], b = s[i0 + stride], c = s[i0 + 2 * stride], e = s[i0 + 3 * stride];
      s[i0] = a + b + c - e;
      s[i0 + stride] = a + b - c + e;
      s[i0 + 2 * stride] = a - b + c + e;
      s[i0 + 3 * stride] = -a + b + c + e;
    }
    stride *= 4;
  }
}

void orc_hadamard256(const float* X, float* Y, int64_t n) { /* app/gpu/kernels.js:360-388 */
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n / 256; g++) {
    float s[256];
    memcpy(s, X + g * 256, sizeof s);
    butterfly256(s);
    for (int j = 0; j < 256; j++) Y[g * 256 + j] = s[j] * 0.0625f;
  }
}

void orc_layernorm_mod(const float* X, const float* MOD, float* Y, int64_t rows, int cols,
                       int64_t shift_off, int64_t scale_off, float eps, int rotate) {
  /* app/gpu/kernels.js:108-145: 256 threads stride the row, 128..1 tree reductions; rows are
   * independent (one per OpenMP thread at a time) */
#pragma omp parallel for schedule(static)
  for (int64_t row = 0; row < rows; row++) {
    float red[256];
    float* S = (float*)malloc(sizeof(float) * (size_t)cols);
    const float* x = X + row * cols;
    for (int t = 0; t < 256; t++) {
      float s = 0.0f;
      for (int c = t; c < cols; c += 256) s += x[c];
      red[t] = s;
    }
    float mean = tree_sum(red, 256) / (float)cols;
    for (int t = 0; t < 256; t++) {
      float v = 0.0f;
      for (int c = t; c < cols; c += 256) {
        float d = x[c] - mean;
        v += d * d;
      }
      red[t] = v;
    }
    float r = 1.0f / sqrtf(tree_sum(red, 256) / (float)cols + eps);
    for (int c = 0; c < cols; c++)
      S[c] = (x[c] - mean) * r * (1.0f + MOD[scale_off + c]) + MOD[shift_off + c];
    if (rotate) {
      for (int g = 0; g < cols / 256; g++) butterfly256(S + g * 256);
      for (int c = 0; c < cols; c++) Y[row * cols + c] = S[c] * 0.0625f;
    } else {
      memcpy(Y + row * cols, S, sizeof(float) * (size_t)cols);
    }
    free(S);
  }
}

/* ------------------------------------------------------------------ attention */

static int kvlen(const orc_attn* a, int b) { return a->kv_len ? a->kv_len[b] : a->Lk; }

void orc_attention_f64(const orc_attn* a) {
  /* (batch, head) pairs are independent: one per thread */
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < a->B; b++)
    for (int h = 0; h < a->H; h++) {
      double* s = (double*)malloc(sizeof(double) * (size_t)a->Lk);
      double* o = (double*)malloc(sizeof(double) * (size_t)a->D);
      const int hk = h / a->group, n = kvlen(a, b);
      for (int i = 0; i < a->Lq; i++) {
        const float* q = a->q + b * a->q_bs + (int64_t)i * a->ldq + a->q_off + (int64_t)h * a->D;
        double mx = -INFINITY;
        for (int j = 0; j < n; j++) {
          const float* k = a->k + b * a->k_bs + (int64_t)j * a->ldk + a->k_off + (int64_t)hk * a->D;
          double acc = 0.0;
          for (int d = 0; d < a->D; d++) acc += (double)q[d] * (double)k[d];
          s[j] = acc * (double)a->scale;
          if (s[j] > mx) mx = s[j];
        }
        double l = 0.0;
        for (int d = 0; d < a->D; d++) o[d] = 0.0;
        for (int j = 0; j < n; j++) {
          double p = exp(s[j] - mx);
          l += p;
          const float* v = a->v + b * a->v_bs + (int64_t)j * a->ldv + a->v_off + (int64_t)hk * a->D;
          for (int d = 0; d < a->D; d++) o[d] += p * (double)v[d];
        }
        float* out = a->o + b * a->o_bs + (int64_t)i * a->ldo + a->o_off + (int64_t)h * a->D;
        for (int d = 0; d < a->D; d++) out[d] = (float)(o[d] / l);
      }
      free(s);
      free(o);
    }
}

void orc_attention_wgsl(const orc_attn* a) {
  /* app/gpu/kernels.js:195-298, one query row at a time; the shader's per-row arithmetic
   * does not depend on the other rows of its workgroup. */
  const int D = a->D;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < a->B; b++)
    for (int h = 0; h < a->H; h++) {
      float s[32], e[32];
      float* o_acc = (float*)malloc(sizeof(float) * (size_t)D);
      const int hk = h / a->group, Lk = kvlen(a, b);
      for (int i = 0; i < a->Lq; i++) {
        const float* q = a->q + b * a->q_bs + (int64_t)i * a->ldq + a->q_off + (int64_t)h * D;
        float m = -1e30f, l = 0.0f;
        for (int d = 0; d < D; d++) o_acc[d] = 0.0f;
        for (int k0 = 0; k0 < Lk; k0 += 32) {
          /* phase 1: s = sum_d q[d] k[d], d in order (kernels.js:206-242) */
          for (int kk = 0; kk < 32; kk++) {
            float acc = 0.0f;
            if (k0 + kk < Lk) {
              const float* k = a->k + b * a->k_bs + (int64_t)(k0 + kk) * a->ldk + a->k_off + (int64_t)hk * D;
              for (int d = 0; d < D; d++) acc += q[d] * k[d];
            }
            s[kk] = acc;
          }
          /* phase 2 (kernels.js:245-272) */
          float bm = -1e30f;
          for (int kk = 0; kk < 32; kk++) {
            float mask = (k0 + kk >= Lk) ? -1e30f : 0.0f;
            s[kk] = s[kk] * a->scale + mask;
            if (s[kk] > bm) bm = s[kk];
          }
          float mn = m > bm ? m : bm;
          for (int kk = 0; kk < 32; kk++) e[kk] = expf(s[kk] - mn);
          float part[8];
          for (int sc = 0; sc < 8; sc++)
            part[sc] = ((e[4 * sc] + e[4 * sc + 1]) + e[4 * sc + 2]) + e[4 * sc + 3];
          float bs = (((part[0] + part[1]) + part[2]) + part[3]) + (((part[4] + part[5]) + part[6]) + part[7]);
          float alpha = expf(m - mn);
          l = l * alpha + bs;
          m = mn;
          for (int d = 0; d < D; d++) o_acc[d] = o_acc[d] * alpha;
          /* phase 3: o += p_k v_k, k in order (kernels.js:276-294) */
          for (int kk = 0; kk < 32; kk++) {
            if (k0 + kk >= Lk) continue; /* the shader loads zero V rows there; p is 0 */
            const float* v = a->v + b * a->v_bs + (int64_t)(k0 + kk) * a->ldv + a->v_off + (int64_t)hk * D;
            for (int d = 0; d < D; d++) o_acc[d] += e[kk] * v[d];
          }
        }
        float inv = 1.0f / l;
        float* out = a->o + b * a->o_bs + (int64_t)i * a->ldo + a->o_off + (int64_t)h * D;
        for (int d = 0; d < D; d++) out[d] = o_acc[d] * inv;
      }
      free(o_acc);
    }
}

float orc_bf16_round(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) { /* NaN stays NaN */
    u |= 0x00400000u;
  } else {
    u = u + 0x7fffu + ((u >> 16) & 1u);
  }
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

void orc_attention_bf16(const orc_attn* a) {
  const int D = a->D;
  const float c = a->scale * 1.4426950408889634f;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < a->B; b++)
    for (int h = 0; h < a->H; h++) {
      float* s = (float*)malloc(sizeof(float) * (size_t)a->Lk);
      float* kb = (float*)malloc(sizeof(float) * (size_t)a->Lk * D);
      float* vb = (float*)malloc(sizeof(float) * (size_t)a->Lk * D);
      double* o = (double*)malloc(sizeof(double) * (size_t)D);
      float* qb = (float*)malloc(sizeof(float) * (size_t)D);
      const int hk = h / a->group, n = kvlen(a, b);
      for (int j = 0; j < n; j++) {
        const float* k = a->k + b * a->k_bs + (int64_t)j * a->ldk + a->k_off + (int64_t)hk * D;
        const float* v = a->v + b * a->v_bs + (int64_t)j * a->ldv + a->v_off + (int64_t)hk * D;
        for (int d = 0; d < D; d++) {
          kb[(size_t)j * D + d] = orc_bf16_round(k[d]);
          vb[(size_t)j * D + d] = orc_bf16_round(v[d]);
        }
      }
      for (int i = 0; i < a->Lq; i++) {
        const float* q = a->q + b * a->q_bs + (int64_t)i * a->ldq + a->q_off + (int64_t)h * D;
        for (int d = 0; d < D; d++) qb[d] = orc_bf16_round(q[d] * c);
        float mx = -INFINITY;
        for (int j = 0; j < n; j++) {
          double acc = 0.0;
          for (int d = 0; d < D; d++) acc += (double)qb[d] * (double)kb[(size_t)j * D + d];
          s[j] = (float)acc;
          if (s[j] > mx) mx = s[j];
        }
        const float m = ceilf(mx);
        double l = 0.0;
        for (int d = 0; d < D; d++) o[d] = 0.0;
        for (int j = 0; j < n; j++) {
          float p = exp2f(s[j] - m);
          double pb = (double)orc_bf16_round(p);
          l += pb;
          for (int d = 0; d < D; d++) o[d] += pb * (double)vb[(size_t)j * D + d];
        }
        float* out = a->o + b * a->o_bs + (int64_t)i * a->ldo + a->o_off + (int64_t)h * D;
        for (int d = 0; d < D; d++) out[d] = (float)(o[d] / l);
      }
      free(s);
      free(kb);
      free(vb);
      free(o);
      free(qb);
    }
}

/* ------------------------------------------------------------------ quantized linears */

void orc_token_quant(const float* X, int64_t M, int K, int8_t* Q, float* S) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; m++) {
    const float* x = X + m * K;
    float amax = 0.0f;
    for (int k = 0; k < K; k++) amax = fmaxf(amax, fabsf(x[k]));
    float s = amax / 127.0f, inv = 127.0f / amax;
    S[m] = s;
    for (int k = 0; k < K; k++) {
      float v = amax == 0.0f ? 0.0f : rintf(x[k] * inv);
      if (v > 127.0f) v = 127.0f;
      if (v < -127.0f) v = -127.0f;
      Q[m * K + k] = (int8_t)v;
    }
  }
}

void orc_gemm_i8(const int8_t* QX, const int8_t* QW, int64_t M, int N, int K, int32_t* ACC) {
  for (int64_t m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      int32_t acc = 0;
      const int8_t* x = QX + m * K;
      const int8_t* w = QW + (int64_t)n * K;
      for (int k = 0; k < K; k++) acc += (int32_t)x[k] * (int32_t)w[k];
      ACC[m * N + n] = acc;
    }
}

float orc_fp8e4m3(uint8_t b) { /* app/gpu/gemm.js:144-151 */
  unsigned e = (b >> 3) & 15u;
  float m = (float)(b & 7u);
  float v = e == 0 ? m * 0.001953125f : (1.0f + m * 0.125f) * ldexpf(1.0f, (int)e - 7);
  return (b & 128u) ? -v : v;
}

void orc_w4_decode(const uint8_t* codes, const uint8_t* srel, const float* cb, int N, int K,
                   int8_t* out) { /* tools/quant.py:172-182; app/gpu/gemm.js:141-158 */
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) {
      uint8_t byte = codes[(int64_t)n * (K / 2) + k / 2];
      int c = (k & 1) ? (byte >> 4) & 15 : byte & 15;
      float s = orc_fp8e4m3(srel[(int64_t)n * (K / 16) + k / 16]);
      float v = rintf(cb[c] * s);
      if (v > 127.0f) v = 127.0f;
      if (v < -127.0f) v = -127.0f;
      out[(int64_t)n * K + k] = (int8_t)v;
    }
}

float orc_gelu(float x) { /* app/gpu/kernels.js:11-18 */
  float z = x * 0.7071067811865476f;
  float s = z > 0.0f ? 1.0f : (z < 0.0f ? -1.0f : 0.0f);
  float a = fabsf(z);
  float t = 1.0f / (1.0f + 0.3275911f * a);
  float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t +
                    0.254829592f) * t * expf(-a * a);
  float erf = s * y;
  return 0.5f * x * (1.0f + erf);
}

float orc_silu(float x) { return x / (1.0f + expf(-x)); } /* app/gpu/kernels.js:19 */

void orc_linear_epilogue(const int32_t* ACC, int64_t M, int N, const float* sx, const float* sw,
                         const float* bias, int act, int epi, const float* gate, int64_t g_off,
                         float* C, int64_t ldc, const float* add) { /* app/gpu/gemm.js:186-192 */
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      float r = (float)ACC[m * N + n];
      if (sx) r = r * sx[m];
      r = r * sw[n];
      if (bias) r = r + bias[n];
      if (add) r = r + add[m * N + n];
      if (act == 1) r = orc_gelu(r);
      if (act == 2) r = orc_silu(r);
      float* c = C + m * ldc + n;
      if (epi == 0) *c = r;
      else if (epi == 1) *c = *c + r;
      else *c = fmaf(gate[g_off + n], r, *c);
    }
}

/* ---------------------------------------------------------------- synthetic weights
 * The seeded fill of anima_fill_random (include/anima.h; no reference counterpart: the reference
 * loads real checkpoints).  splitmix64 is Vigna's published generator (xoshiro/splitmix64.c);
 * the FP kinds round every product and sum (no contraction), as the device code does. */
static uint64_t orc_splitmix64(uint64_t x) {
  uint64_t z = x + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t orc_splitmix64_next(uint64_t state) { return orc_splitmix64(state); }

static uint16_t orc_bf16_bits(float v) { /* round to nearest even (finite inputs) */
  uint32_t u;
  memcpy(&u, &v, 4);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

void orc_fill_random(void* dst, int64_t n, int kind, uint64_t seed, float lo, float hi) {
  const int64_t imul = (int64_t)llrint((double)lo * 4096.0 / 147.8017);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) {
    const uint64_t h = orc_splitmix64(seed * 0xD1B54A32D192ED03ull + (uint64_t)i);
    if (kind == 0) { /* U8 */
      const int64_t a = (int64_t)lo, b = (int64_t)hi;
      ((uint8_t*)dst)[i] = (uint8_t)(a + (int64_t)(h % (uint64_t)(b - a + 1)));
    } else if (kind == 1) { /* I8N */
      const int64_t sum = (int64_t)(h & 0xff) + (int64_t)((h >> 8) & 0xff) + (int64_t)((h >> 16) & 0xff) +
                          (int64_t)((h >> 24) & 0xff);
      int64_t v = ((sum - 510) * imul) >> 12;
      v = v < -127 ? -127 : (v > 127 ? 127 : v);
      ((int8_t*)dst)[i] = (int8_t)v;
    } else if (kind == 4) { /* F32N */
      const float u = (float)(h & 0xffff) * (1.0f / 65536.0f) + (float)((h >> 16) & 0xffff) * (1.0f / 65536.0f) +
                      (float)((h >> 32) & 0xffff) * (1.0f / 65536.0f) + (float)((h >> 48) & 0xffff) * (1.0f / 65536.0f);
      ((float*)dst)[i] = (u - 2.0f) * 1.7320508f * lo + hi;
    } else { /* F32, BF16 */
      const float u = (float)(h >> 40) * (1.0f / 16777216.0f);
      const float v = lo + (hi - lo) * u;
      if (kind == 2) ((float*)dst)[i] = v;
      else ((uint16_t*)dst)[i] = orc_bf16_bits(v);
    }
  }
}

/* ---------------------------------------------------------------- VAE */
void orc_channel_norm(const float* X, const float* G, float* Y, int64_t rows, int cols, int silu) {
  /* app/gpu/kernels.js:65-89 mode 1: 64 threads stride the row, then the 32 .. 1 tree */
#pragma omp parallel for schedule(static)
  for (int64_t row = 0; row < rows; row++) {
    const float* x = X + row * cols;
    float red[64];
    for (int t = 0; t < 64; t++) {
      float ss = 0.0f;
      for (int c = t; c < cols; c += 64) ss += x[c] * x[c];
      red[t] = ss;
    }
    for (int s = 32; s > 0; s >>= 1)
      for (int t = 0; t < s; t++) red[t] = red[t] + red[t + s];
    const float r = sqrtf((float)cols) / fmaxf(sqrtf(red[0]), 1e-12f);
    for (int c = 0; c < cols; c++) {
      float y = x[c] * r * G[c];
      if (silu) y = y / (1.0f + expf(-y));
      Y[row * cols + c] = y;
    }
  }
}
