// Tiled bf16-MFMA GEMM for fp32 activations, and what the VAE decoder builds on it:
//   * conv3x3 (pad 1) of an NHWC image as an implicit GEMM, with the 2x nearest upsample of the
//     input fused into the operand loads and the residual add into the epilogue (the "conv3" loader
//     of app/gpu/gemm.js:56-80, dispatched by ops.conv3x3 / conv3x3Into, app/gpu/ops.js:95-109);
//   * the Wan channel norm y = x / max(||x||, 1e-12) * sqrt(C) * gamma (+ SiLU) of
//     app/gpu/kernels.js:62-89 (mode 1), in the shader's reduction order;
//   * attention for head dims other than 128 (the LLM adapter's 64, the VAE's single 384-dim head),
//     on the reference's chunked path (app/gpu/ops.js:177-207): scores for a chunk of query rows, a
//     row softmax (optionally causal), then P.V.
//
// The GEMM: C[m][n] = alpha * sum_k A[m][k] B[n][k] (* rs[m]) (+ bias[n]) (act), stored or added
// to C.  One workgroup = 4 waves = a 128 x 128 output tile, each wave 64 x 64 (2 x 2 tiles of
// v_mfma_f32_32x32x16_bf16); k-tiles of 32 are converted to bf16 while they move from global
// memory into a double-buffered LDS image (one barrier per k-tile, the next tile's global loads
// issued before the current tile's MFMAs).  fp32 operands are rounded to bf16, or, with SPLIT,
// written as two bf16 terms x = hi + lo (lo = bf16(x - hi), exact difference): the products
// hi.hi + lo.hi (+ hi.lo for an fp32 B) then carry about 16 significant bits of each operand, an
// fp32-level result (relative error ~1e-5 over long sums) from the bf16 matrix cores.  bf16
// weights (the VAE's checkpoint format) are exact and never split.
#include <algorithm>
#include <cmath>

#include "common.h"
#include "internal.h"

namespace anima {

constexpr int TG_BM = 128, TG_BN = 128, TG_BK = 32;
constexpr int TG_ROW = TG_BK + 8;  // LDS row stride in bf16 (80 B): conflict-free fragment reads

enum { TG_A_ROWS = 0, TG_A_CONV = 1 };
enum { TG_B_W16 = 0, TG_B_F32 = 1 };

struct TGemmArgs {
  // A: a[z*a_bs + m*lda + k], or (conv) the im2col of the NHWC image a[z*a_bs + ((b*Hin + y)*Win + x)*cin + c]
  const float* a;
  int64_t lda, a_bs;
  int cin, H, W, up;  // conv: output H x W per image; the input is H x W, or H/2 x W/2 with up
  // B: b[z*b_bs + n*ldb + k], bf16 or fp32
  const void* b;
  int64_t ldb, b_bs;
  float* c;
  int64_t ldc, c_bs;
  const float* bias;  // [N] or null
  const float* rs;    // per-row scale rs[z*rs_bs + m] or null
  int64_t rs_bs;
  float alpha;
  int act, resid;
  int M, N, K;
};

// The output pixel of a conv A row, decomposed once per thread: image base pointer and (oy, ox).
struct ConvRow {
  const float* img;  // first element of this row's image
  int oy, ox;
};

__device__ __forceinline__ ConvRow conv_row(const TGemmArgs& p, const float* a, int m) {
  ConvRow r;
  const int hw = p.H * p.W;
  const int img = m / hw, q = m - img * hw;
  r.oy = q / p.W;
  r.ox = q - r.oy * p.W;
  const int Hin = p.up ? p.H >> 1 : p.H, Win = p.up ? p.W >> 1 : p.W;
  r.img = a + (int64_t)img * Hin * Win * p.cin;
  return r;
}

// 16 consecutive k of A row m starting at k (k % 16 == 0), fp32; zeros outside the matrix / image.
template <int AM>
__device__ __forceinline__ void tg_load_a(const TGemmArgs& p, const float* a, const ConvRow& cr, int m, int k,
                                          float (&v)[16]) {
  bool ok = m < p.M && k < p.K;
  const float* src = nullptr;
  if (ok) {
    if constexpr (AM == TG_A_ROWS) {
      src = a + (int64_t)m * p.lda + k;
    } else {
      const int tap = k / p.cin, ci = k - tap * p.cin;  // cin is uniform: a scalar division
      const int ty = tap / 3, tx = tap - 3 * ty;
      const int iy = cr.oy + ty - 1, ix = cr.ox + tx - 1;
      ok = iy >= 0 && ix >= 0 && iy < p.H && ix < p.W;
      const int Win = p.up ? p.W >> 1 : p.W;
      const int sy = p.up ? iy >> 1 : iy, sx = p.up ? ix >> 1 : ix;
      src = cr.img + ((int64_t)sy * Win + sx) * p.cin + ci;
    }
  }
  if (ok && (AM == TG_A_CONV || k + 16 <= p.K)) {  // conv: cin % 16 == 0, a run never crosses a tap
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 t = *(const float4*)(src + 4 * j);
      v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
    }
  } else if (ok) {  // rows: the last, partial k-run
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = k + j < p.K ? src[j] : 0.0f;
  } else {
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = 0.0f;
  }
}

__device__ __forceinline__ void tg_split(const float (&v)[16], bf16x8 (&hi)[2], bf16x8 (&lo)[2], bool split) {
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const bf16 h = to_bf16(v[j]);
    hi[j >> 3][j & 7] = h;
    if (split) lo[j >> 3][j & 7] = to_bf16(v[j] - (float)h);
  }
}

template <int AM, int BMODE, bool SPLIT>
__global__ __launch_bounds__(256) void tgemm_kernel(TGemmArgs p) {
  constexpr int NA = SPLIT ? 2 : 1;
  constexpr int NB = (SPLIT && BMODE == TG_B_F32) ? 2 : 1;
  __shared__ __attribute__((aligned(16))) bf16 sa[2][NA][TG_BM * TG_ROW];
  __shared__ __attribute__((aligned(16))) bf16 sb[2][NB][TG_BN * TG_ROW];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lq = lane & 31, hf = lane >> 5;
  const int z = blockIdx.z;
  const int m0 = blockIdx.x * TG_BM, n0 = blockIdx.y * TG_BN;
  const float* a = p.a + (int64_t)z * p.a_bs;
  const char* bb = (const char*)p.b + (int64_t)z * p.b_bs * (BMODE == TG_B_W16 ? 2 : 4);
  // loader role: row t/2 of the A and B tiles, k-half t%2 (16 k)
  const int lr = tid >> 1, lk = 16 * (tid & 1);
  const int am = m0 + lr, bn = n0 + lr;
  const bool bok = bn < p.N;

  ConvRow cr{};
  if constexpr (AM == TG_A_CONV) {
    if (am < p.M) cr = conv_row(p, a, am);
  }
  float av[16];
  uint4 bw[2];   // bf16 B: 16 values
  float bv[16];  // fp32 B
  auto load = [&](int k0) {
    tg_load_a<AM>(p, a, cr, am, k0 + lk, av);
    const int k = k0 + lk;
    if constexpr (BMODE == TG_B_W16) {
      const uint16_t* src = (const uint16_t*)bb + (int64_t)bn * p.ldb + k;
      if (bok && k + 16 <= p.K) {
        bw[0] = *(const uint4*)src;
        bw[1] = *(const uint4*)(src + 8);
      } else {
        uint16_t t[16];
#pragma unroll
        for (int j = 0; j < 16; j++) t[j] = bok && k + j < p.K ? src[j] : (uint16_t)0;
        uint32_t u[8];
#pragma unroll
        for (int j = 0; j < 8; j++) u[j] = (uint32_t)t[2 * j] | ((uint32_t)t[2 * j + 1] << 16);
        bw[0] = make_uint4(u[0], u[1], u[2], u[3]);
        bw[1] = make_uint4(u[4], u[5], u[6], u[7]);
      }
    } else {
      const float* src = (const float*)bb + (int64_t)bn * p.ldb + k;
      if (bok && k + 16 <= p.K) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float4 t = *(const float4*)(src + 4 * j);
          bv[4 * j] = t.x; bv[4 * j + 1] = t.y; bv[4 * j + 2] = t.z; bv[4 * j + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; j++) bv[j] = bok && k + j < p.K ? src[j] : 0.0f;
      }
    }
  };
  auto store = [&](int st) {
    bf16x8 hi[2], lo[2];
    tg_split(av, hi, lo, SPLIT);
    *(bf16x8*)(&sa[st][0][lr * TG_ROW + lk]) = hi[0];
    *(bf16x8*)(&sa[st][0][lr * TG_ROW + lk + 8]) = hi[1];
    if constexpr (SPLIT) {
      *(bf16x8*)(&sa[st][NA - 1][lr * TG_ROW + lk]) = lo[0];
      *(bf16x8*)(&sa[st][NA - 1][lr * TG_ROW + lk + 8]) = lo[1];
    }
    if constexpr (BMODE == TG_B_W16) {
      *(uint4*)(&sb[st][0][lr * TG_ROW + lk]) = bw[0];
      *(uint4*)(&sb[st][0][lr * TG_ROW + lk + 8]) = bw[1];
    } else {
      bf16x8 bh[2], bl[2];
      tg_split(bv, bh, bl, NB == 2);
      *(bf16x8*)(&sb[st][0][lr * TG_ROW + lk]) = bh[0];
      *(bf16x8*)(&sb[st][0][lr * TG_ROW + lk + 8]) = bh[1];
      if constexpr (NB == 2) {
        *(bf16x8*)(&sb[st][NB - 1][lr * TG_ROW + lk]) = bl[0];
        *(bf16x8*)(&sb[st][NB - 1][lr * TG_ROW + lk + 8]) = bl[1];
      }
    }
  };

  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f32x16{};

  const int nkt = (p.K + TG_BK - 1) / TG_BK;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; kt++) {
    const int st = kt & 1;
    if (kt + 1 < nkt) load((kt + 1) * TG_BK);
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      bf16x8 fa[2][NA], fb[2][NB];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int r = (64 * wm + 32 * i + lq) * TG_ROW + 16 * ks + 8 * hf;
#pragma unroll
        for (int s = 0; s < NA; s++) fa[i][s] = *(const bf16x8*)(&sa[st][s][r]);
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int r = (64 * wn + 32 * j + lq) * TG_ROW + 16 * ks + 8 * hf;
#pragma unroll
        for (int s = 0; s < NB; s++) fb[j][s] = *(const bf16x8*)(&sb[st][s][r]);
      }
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][0], fb[j][0], acc[i][j], 0, 0, 0);
          if constexpr (SPLIT) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][1], fb[j][0], acc[i][j], 0, 0, 0);
            if constexpr (NB == 2) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][0], fb[j][1], acc[i][j], 0, 0, 0);
          }
        }
    }
    if (kt + 1 < nkt) store(st ^ 1);
    __syncthreads();
  }

  // epilogue: register r of tile (i, j) holds row 8(r/4) + 4hf + r%4 and column lq of the tile
  float* cz = p.c + (int64_t)z * p.c_bs;
  const float* rs = p.rs ? p.rs + (int64_t)z * p.rs_bs : nullptr;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = n0 + 64 * wn + 32 * j + lq;
    if (n >= p.N) continue;
    const float bias = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (m >= p.M) continue;
        float v = acc[i][j][r] * p.alpha;
        if (rs) v = v * rs[m];
        v = v + bias;
        if (p.act == ANIMA_ACT_SILU) v = silu_f(v);
        else if (p.act == ANIMA_ACT_GELU) v = gelu_erf(v);
        float* dst = cz + (int64_t)m * p.ldc + n;
        *dst = p.resid ? *dst + v : v;
      }
  }
}

// Launches tgemm_kernel over a batch of `batch` independent products (blockIdx.z).
static int tgemm_launch(anima_ctx* c, const TGemmArgs& p, int amode, int bmode, bool split, int batch, const char* name,
                        double flops) {
  if (p.M <= 0 || p.N <= 0 || p.K <= 0 || batch <= 0) return ANIMA_OK;
  const int64_t gn = (p.N + TG_BN - 1) / TG_BN;
  if (gn > 65535 || batch > 65535) return fail(c, ANIMA_E_ARG, "%s: N=%d, batch %d beyond the grid", name, p.N, batch);
  dim3 grid((p.M + TG_BM - 1) / TG_BM, (unsigned)gn, batch);
  Launch L(c, name, flops, 0.0);
#define TG(A, B, S) hipLaunchKernelGGL((tgemm_kernel<A, B, S>), grid, dim3(256), 0, c->stream, p)
  if (amode == TG_A_CONV) {
    if (split) TG(TG_A_CONV, TG_B_W16, true);
    else TG(TG_A_CONV, TG_B_W16, false);
  } else if (bmode == TG_B_W16) {
    if (split) TG(TG_A_ROWS, TG_B_W16, true);
    else TG(TG_A_ROWS, TG_B_W16, false);
  } else {
    if (split) TG(TG_A_ROWS, TG_B_F32, true);
    else TG(TG_A_ROWS, TG_B_F32, false);
  }
#undef TG
  return L.end();
}

// ---- conv3x3 on spatial tiles: a workgroup (8 waves) computes a 16 x 32 block of output pixels
// for BN = 96 output channels (or one 32-wide column tile when cout <= 32: the 3-channel head).  Per step of 32 input channels the input halo it needs (18 x 34 pixels in
// output coordinates, sampled through the 2x nearest upsample when up; zero outside the image) and
// the 9 x 96 x 32 weights are copied once into LDS, so every input value is read from memory once
// per step instead of once per tap (the row-tiled implicit GEMM reads each pixel nine times).  The
// next step's halo and weights are loaded into registers before this step's MFMAs.  With NW waves,
// wave w owns MT = 16 / NW output rows from MT w (32-pixel MFMA row tiles) x three 32-channel
// column tiles (NW = 8: 4 waves ran the fp32 convs 10-15% slower and the bf16 ones 2% faster); for tap
// (ty, tx) the A row of output pixel (r, c) is halo pixel (r + ty, c + tx).  LDS rows are 64 bytes
// (32 channels) with the 16-byte unit u of row q stored at slot u ^ ((q / 4) % 4), so the fragment
// reads of 16 consecutive rows fall in distinct bank groups.  Products and sums are those of
// tgemm_kernel (activation rounded to bf16, or split hi + lo with SPLIT; bf16 weights exact); only
// the order of the k-terms differs (input-channel chunk outer, tap inner).
constexpr int CT_TH = 16, CT_TW = 32, CT_HH = CT_TH + 2, CT_HW = CT_TW + 2, CT_HP = CT_HH * CT_HW;
constexpr int CT_CC = 32, CT_NW = 8;
constexpr int CT_HU = CT_HP * 4;          // 16-byte units of one halo plane (8 channels each)

__device__ __forceinline__ int ct_off(int row, int u) { return row * 64 + ((u ^ ((row >> 2) & 3)) << 4); }

template <bool SPLIT, int NW, int BN>
__global__ __launch_bounds__(64 * NW) void conv3x3_tile_kernel(TGemmArgs p) {
  constexpr int NA = SPLIT ? 2 : 1;
  constexpr int NJ = BN / 32;              // 32-channel MFMA column tiles per wave
  constexpr int CT_WU = 9 * BN * 4;        // 16-byte units of the step's weights
  constexpr int NT = 64 * NW, MT = CT_TH / NW;  // threads; output rows (32-pixel MFMA tiles) per wave
  constexpr int CT_HJ = (CT_HU + NT - 1) / NT, CT_WJ = (CT_WU + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) char lds[NA * CT_HP * 64 + 9 * BN * 64];
  char* const wl = lds + NA * CT_HP * 64;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, lq = lane & 31, hf = lane >> 5;
  const int tx_n = p.W / CT_TW, ty_n = p.H / CT_TH;
  const int tile = blockIdx.x, img = tile / (tx_n * ty_n), trem = tile - img * tx_n * ty_n;
  const int oy0 = (trem / tx_n) * CT_TH, ox0 = (trem % tx_n) * CT_TW;
  const int n0 = blockIdx.y * BN;
  const int Hin = p.up ? p.H >> 1 : p.H, Win = p.up ? p.W >> 1 : p.W;
  const float* imgp = p.a + (int64_t)img * Hin * Win * p.cin;
  const uint16_t* W = (const uint16_t*)p.b;

  // staged loads of one step (input channels c0 .. c0 + 31); addresses past the image or the
  // unit count are clamped to valid memory and their units stored as zeros / skipped
  float4 hv[CT_HJ][2];
  uint4 wv[CT_WJ];
  unsigned hok = 0;
  auto stage = [&](int c0) {
    hok = 0;
#pragma unroll
    for (int j = 0; j < CT_HJ; j++) {
      const int U = t + NT * j, px = min(U, CT_HU - 1) >> 2, u = U & 3;
      const int hy = px / CT_HW, hx = px - hy * CT_HW;
      const int y = oy0 - 1 + hy, x = ox0 - 1 + hx;
      const bool ok = U < CT_HU && y >= 0 && x >= 0 && y < p.H && x < p.W;
      const int sy = ok ? (p.up ? y >> 1 : y) : 0, sx = ok ? (p.up ? x >> 1 : x) : 0;
      const float* src = imgp + ((int64_t)sy * Win + sx) * p.cin + c0 + 8 * u;
      hv[j][0] = *(const float4*)src;
      hv[j][1] = *(const float4*)(src + 4);
      hok |= (ok ? 1u : 0u) << j;
    }
#pragma unroll
    for (int j = 0; j < CT_WJ; j++) {
      const int V = min(t + NT * j, CT_WU - 1), tap = V / (BN * 4), rem = V - tap * BN * 4;
      const int n = min(n0 + (rem >> 2), p.N - 1), u = rem & 3;  // channels past cout: never stored
      wv[j] = *(const uint4*)(W + (int64_t)n * p.ldb + tap * p.cin + c0 + 8 * u);
    }
  };
  auto publish = [&]() {
#pragma unroll
    for (int j = 0; j < CT_HJ; j++) {
      const int U = t + NT * j;
      if (U >= CT_HU) break;
      const int px = U >> 2, u = U & 3;
      const bool ok = (hok >> j) & 1;
      const float v[8] = {hv[j][0].x, hv[j][0].y, hv[j][0].z, hv[j][0].w, hv[j][1].x, hv[j][1].y, hv[j][1].z, hv[j][1].w};
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float f = ok ? v[e] : 0.0f;
        hi[e] = to_bf16(f);
        if (SPLIT) lo[e] = to_bf16(f - (float)hi[e]);
      }
      *(bf16x8*)(lds + ct_off(px, u)) = hi;
      if constexpr (SPLIT) *(bf16x8*)(lds + CT_HP * 64 + ct_off(px, u)) = lo;
    }
#pragma unroll
    for (int j = 0; j < CT_WJ; j++) {
      const int V = t + NT * j;
      if (V >= CT_WU) break;
      const int tap = V / (BN * 4), rem = V - tap * BN * 4;
      *(uint4*)(wl + ct_off(tap * BN + (rem >> 2), rem & 3)) = wv[j];
    }
  };

  f32x16 acc[MT][NJ];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = f32x16{};

  stage(0);
  for (int c0 = 0; c0 < p.cin; c0 += CT_CC) {
    if (c0 > 0) __syncthreads();  // every wave is done with the previous step's tiles
    publish();
    __syncthreads();
    stage(min(c0 + CT_CC, p.cin - CT_CC));  // the next step's loads fly during these MFMAs
#pragma unroll
    for (int tap = 0; tap < 9; tap++) {
      const int ty = tap / 3, tx = tap - 3 * ty;
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const int u = 2 * s + hf;
        bf16x8 fa[MT][NA], fb[NJ];
#pragma unroll
        for (int i = 0; i < MT; i++) {
          const int px = (MT * wave + i + ty) * CT_HW + lq + tx;
#pragma unroll
          for (int a = 0; a < NA; a++) fa[i][a] = *(const bf16x8*)(lds + a * CT_HP * 64 + ct_off(px, u));
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) fb[j] = *(const bf16x8*)(wl + ct_off(tap * BN + 32 * j + lq, u));
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
          for (int j = 0; j < NJ; j++) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][0], fb[j], acc[i][j], 0, 0, 0);
            if constexpr (SPLIT) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][1], fb[j], acc[i][j], 0, 0, 0);
          }
      }
    }
  }

  // epilogue: register r of tile (i, j) holds pixel 8(r/4) + 4hf + r%4 of output row oy0 + 2w + i
  // and channel n0 + 32j + lq
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int n = n0 + 32 * j + lq;
    if (n >= p.N) continue;
    const float bias = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < MT; i++) {
      const int y = oy0 + MT * wave + i;
      float* orow = p.c + (((int64_t)img * p.H + y) * p.W + ox0) * p.ldc + n;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int x = 8 * (r >> 2) + 4 * hf + (r & 3);
        float v = acc[i][j][r] * p.alpha;
        v = v + bias;
        float* dst = orow + (int64_t)x * p.ldc;
        *dst = p.resid ? *dst + v : v;
      }
    }
  }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int conv3x3_launch(anima_ctx* c, const anima_conv_desc* d) {
  if (!d) return fail(c, ANIMA_E_ARG, "anima_conv3x3: null descriptor");
  if (!d->x || !d->w || !d->out) return fail(c, ANIMA_E_ARG, "anima_conv3x3: null x / w / out");
  if (d->B < 1 || d->H < 1 || d->W < 1 || d->cin < 1 || d->cout < 1)
    return fail(c, ANIMA_E_ARG, "anima_conv3x3: B=%d H=%d W=%d cin=%d cout=%d", d->B, d->H, d->W, d->cin, d->cout);
  if (d->cin % 16) return fail(c, ANIMA_E_UNSUPPORTED, "anima_conv3x3: cin=%d (this build needs cin %% 16 == 0)", d->cin);
  if (d->up && (d->H % 2 || d->W % 2)) return fail(c, ANIMA_E_ARG, "anima_conv3x3: up needs an even output size (H=%d W=%d)", d->H, d->W);
  if (d->precision != ANIMA_PREC_BF16 && d->precision != ANIMA_PREC_FP32)
    return fail(c, ANIMA_E_ARG, "anima_conv3x3: unknown precision %d", d->precision);
  if (!al16(d->x) || !al16(d->w)) return fail(c, ANIMA_E_ARG, "anima_conv3x3: x and w must be 16-byte aligned");
  const int64_t M = (int64_t)d->B * d->H * d->W;
  if (M > 0x7fffffffLL - TG_BM) return fail(c, ANIMA_E_ARG, "anima_conv3x3: %lld output pixels", (long long)M);
  TGemmArgs p{};
  p.a = d->x;
  p.cin = d->cin;
  p.H = d->H;
  p.W = d->W;
  p.up = d->up ? 1 : 0;
  p.b = d->w;
  p.ldb = 9LL * d->cin;
  p.c = d->out;
  p.ldc = d->cout;
  p.bias = d->bias;
  p.alpha = 1.0f;
  p.act = ANIMA_ACT_NONE;
  p.resid = d->resid ? 1 : 0;
  p.M = (int)M;
  p.N = d->cout;
  p.K = 9 * d->cin;
  const bool split = d->precision == ANIMA_PREC_FP32;
  const int bn = d->cout % 96 == 0 ? 96 : d->cout <= 32 ? 32 : 0;  // 96-channel tiles, or one 32-wide tile
  if (bn && d->cin % CT_CC == 0 && d->H % CT_TH == 0 && d->W % CT_TW == 0 &&
      (int64_t)d->B * (d->H / CT_TH) * (d->W / CT_TW) <= 0x7fffffff && (d->cout + bn - 1) / bn <= 65535) {
    // spatial tiles with the input halo in LDS
    const dim3 grid((unsigned)((int64_t)d->B * (d->H / CT_TH) * (d->W / CT_TW)), (unsigned)((d->cout + bn - 1) / bn));
    Launch L(c, d->up ? "conv3x3.up" : "conv3x3", 2.0 * M * d->cout * 9.0 * d->cin, 0.0);
#define CTL(S, BN) hipLaunchKernelGGL((conv3x3_tile_kernel<S, CT_NW, BN>), grid, dim3(64 * CT_NW), 0, c->stream, p)
    if (bn == 96) {
      if (split) CTL(true, 96);
      else CTL(false, 96);
    } else {
      if (split) CTL(true, 32);
      else CTL(false, 32);
    }
#undef CTL
    return L.end();
  }
  return tgemm_launch(c, p, TG_A_CONV, TG_B_W16, split, 1, d->up ? "conv3x3.up" : "conv3x3",
                      2.0 * M * d->cout * 9.0 * d->cin);
}

// ---- channel norm: one wave per row; lane t sums x[c]^2 over c = t, t + 64, ... in order, then the
// 32 .. 1 tree of the shader's shared-memory reduction (kernels.js:78-79).
__global__ __launch_bounds__(256) void channel_norm_kernel(const float* X, const float* G, float* Y, int64_t rows, int cols,
                                                           int silu) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* x = X + row * cols;
  float ss = 0.0f;
  for (int c = lane; c < cols; c += 64) ss += x[c] * x[c];
  ss = tree_sum_down(ss, 64);
  const float r = sqrtf((float)cols) / fmaxf(sqrtf(__shfl(ss, 0)), 1e-12f);
  float* y = Y + row * cols;
  for (int c = lane; c < cols; c += 64) {
    float v = x[c] * r * G[c];
    if (silu) v = silu_f(v);
    y[c] = v;
  }
}

// The same per-row arithmetic for rows of at most 64 NV channels, CN_RPW rows per wave with every
// load of the wave issued first: one row per wave kept too few bytes in flight (a row of 96
// channels is 384 bytes) and left the pass at a third of the HBM rate.  Channels past cols read as
// zero, which adds nothing to a lane's sum (0 + x^2 and x^2 + 0 are exact).
constexpr int CN_RPW = 8;
template <int NV>
__global__ __launch_bounds__(256) void channel_norm_rows_kernel(const float* X, const float* G, float* Y, int64_t rows,
                                                                int cols, int silu) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * CN_RPW;
  float xv[CN_RPW][NV], g[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int c = lane + 64 * v;
    g[v] = c < cols ? G[c] : 0.0f;
  }
#pragma unroll
  for (int r = 0; r < CN_RPW; r++)
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int c = lane + 64 * v;
      xv[r][v] = row0 + r < rows && c < cols ? X[(row0 + r) * cols + c] : 0.0f;
    }
#pragma unroll
  for (int r = 0; r < CN_RPW; r++) {
    if (row0 + r >= rows) break;  // uniform across the wave
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; v++) ss += xv[r][v] * xv[r][v];
    ss = tree_sum_down(ss, 64);
    const float rn = sqrtf((float)cols) / fmaxf(sqrtf(__shfl(ss, 0)), 1e-12f);
    float* y = Y + (row0 + r) * cols;
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int c = lane + 64 * v;
      float o = xv[r][v] * rn * g[v];
      if (silu) o = silu_f(o);
      if (c < cols) y[c] = o;
    }
  }
}

int channel_norm_launch(anima_ctx* c, const float* x, const float* gamma, float* y, int64_t rows, int cols, int silu) {
  if (!x || !gamma || !y) return fail(c, ANIMA_E_ARG, "anima_channel_norm: null pointer");
  if (rows < 0 || cols < 1) return fail(c, ANIMA_E_ARG, "anima_channel_norm: rows=%lld cols=%d", (long long)rows, cols);
  if (rows == 0) return ANIMA_OK;
  Launch lc(c, "vae.channel_norm", 0.0, (double)rows * cols * 8);
  const unsigned gr = (unsigned)((rows + 4 * CN_RPW - 1) / (4 * CN_RPW));
  const int sl = silu ? 1 : 0;
  if (cols <= 128) hipLaunchKernelGGL(channel_norm_rows_kernel<2>, dim3(gr), dim3(256), 0, c->stream, x, gamma, y, rows, cols, sl);
  else if (cols <= 192) hipLaunchKernelGGL(channel_norm_rows_kernel<3>, dim3(gr), dim3(256), 0, c->stream, x, gamma, y, rows, cols, sl);
  else if (cols <= 384) hipLaunchKernelGGL(channel_norm_rows_kernel<6>, dim3(gr), dim3(256), 0, c->stream, x, gamma, y, rows, cols, sl);
  else
    hipLaunchKernelGGL(channel_norm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, c->stream, x, gamma, y, rows,
                       cols, sl);
  return lc.end();
}

// ---- the decoder's output image (app/models/vae.js:104-112): RGBA bytes of [n][3] values,
// channel = round((clamp(v, -1, 1) + 1) / 2 * 255) in double precision with JS Math.round
// (nearest, ties toward +inf; t - floor(t) is exact in double), NaN -> 0 as the reference's
// Uint8ClampedArray store makes it, alpha 255.
__global__ __launch_bounds__(256) void rgba_kernel(const float* x, int64_t n, uint8_t* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  uchar4 o;
  unsigned char c[3];
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const float xv = x[3 * i + j];
    const double v = (fmin(1.0, fmax(-1.0, (double)xv)) + 1.0) / 2.0;
    const double t = v * 255.0;
    double r = floor(t);
    if (t - r >= 0.5) r += 1.0;
    c[j] = xv != xv ? 0 : (unsigned char)r;
  }
  o.x = c[0];
  o.y = c[1];
  o.z = c[2];
  o.w = 255;
  ((uchar4*)out)[i] = o;
}

int to_rgba_launch(anima_ctx* c, const float* x, int64_t n, uint8_t* out) {
  if (!x || !out || n < 0) return fail(c, ANIMA_E_ARG, "anima_to_rgba: bad arguments");
  if (((uintptr_t)out & 3) != 0) return fail(c, ANIMA_E_ARG, "anima_to_rgba: out must be 4-byte aligned");
  if (n == 0) return ANIMA_OK;
  Launch l(c, "vae.to_rgba", 0.0, (double)n * 16);
  hipLaunchKernelGGL(rgba_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, c->stream, x, n, out);
  return l.end();
}

// ---- attention on the chunked path (head dims other than 64 / 128)

// In place on row r of S (row stride ld), columns [0, cols): e = exp(s * scale - m), m the maximum of
// s * scale over the row's first `lim` columns, 0 past them; rl[r] = 1 / sum of e (the P.V
// product's row scale).  lim = valid, or with the causal mask (app/gpu/kernels.js:49,
// limit = min(cols, row + 1)) min(valid, q + 1) for the row's query index q = row0 + r.  One
// workgroup per row.
__global__ __launch_bounds__(256) void chunk_softmax_kernel(float* S, int64_t ld, float* rl, int cols, int valid,
                                                            float scale, int row0, int causal) {
  __shared__ float red[4];
  float* s = S + (int64_t)blockIdx.x * ld;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int lim = causal ? min(valid, row0 + (int)blockIdx.x + 1) : valid;
  float mx = -INFINITY;
  for (int c = t; c < lim; c += 256) mx = fmaxf(mx, s[c] * scale);
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.0f;
  for (int c = t; c < cols; c += 256) {
    const float e = c < lim ? expf(s[c] * scale - mx) : 0.0f;
    s[c] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  if (t == 0) rl[blockIdx.x] = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
}

// The same row softmax with the row held in registers (NPT values per thread, columns t + 256 i):
// one read and one write of the score row instead of two reads and a write; the maximum, the
// exponentials and the sums are taken in the same order as chunk_softmax_kernel (bit-identical).
template <int NPT>
__global__ __launch_bounds__(256) void chunk_softmax_reg_kernel(float* S, int64_t ld, float* rl, int cols, int valid,
                                                                float scale, int row0, int causal) {
  __shared__ float red[4];
  float* s = S + (int64_t)blockIdx.x * ld;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int lim = causal ? min(valid, row0 + (int)blockIdx.x + 1) : valid;
  float v[NPT];
#pragma unroll
  for (int i = 0; i < NPT; i++) {
    const int c = t + 256 * i;
    v[i] = c < cols ? s[c] : 0.0f;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NPT; i++)
    if (t + 256 * i < lim) mx = fmaxf(mx, v[i] * scale);
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < NPT; i++) {
    const int c = t + 256 * i;
    if (c < cols) {
      const float e = c < lim ? expf(v[i] * scale - mx) : 0.0f;
      s[c] = e;
      sum += e;
    }
  }
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  if (t == 0) rl[blockIdx.x] = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
}

// dst[d * ldd + j] = src[j * ld + d] for j < L, d < D (V -> V^T for the P.V product's B operand).
__global__ __launch_bounds__(256) void transpose_kernel(const float* src, int64_t ld, int L, int D, float* dst, int64_t ldd) {
  __shared__ float tile[32][33];
  const int j0 = blockIdx.x * 32, d0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8) {
    const int j = j0 + r, d = d0 + tx;
    tile[r][tx] = j < L && d < D ? src[(int64_t)j * ld + d] : 0.0f;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int d = d0 + r, j = j0 + tx;
    if (d < D && j < L) dst[(int64_t)d * ldd + j] = tile[tx][r];
  }
}

// Checks of the chunked path: plain attention (no fused norm / RoPE, no prepared K/V; causal mask
// allowed) with 16-byte aligned rows, D % 4 == 0.
int attention_chunked_check(anima_ctx* c, const anima_attn_desc* d) {
  if (d->D < 4 || d->D % 4 || d->D > 4096)
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention: head dim %d (the chunked path takes D %% 4 == 0, D <= 4096)", d->D);
  if (d->q_norm || d->k_norm || d->rope_cs || d->kv_prep)
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention: head dim %d takes no fused norm / RoPE or prepared K/V", d->D);
  if (d->precision != ANIMA_PREC_BF16 && d->precision != ANIMA_PREC_FP32)
    return fail(c, ANIMA_E_ARG, "anima_attention: unknown precision %d", d->precision);
  const int group = d->group <= 0 ? 1 : d->group;
  if (d->B < 1 || d->Lq < 1 || d->Lk < 1 || d->H < 1 || d->H % group)
    return fail(c, ANIMA_E_ARG, "anima_attention: B=%d Lq=%d Lk=%d H=%d group=%d", d->B, d->Lq, d->Lk, d->H, group);
  if (!d->q || !d->k || !d->v || !d->o) return fail(c, ANIMA_E_ARG, "anima_attention: null q/k/v/o");
  const int64_t lds[4] = {d->ldq, d->ldk, d->ldv, d->ldo}, offs[4] = {d->q_off, d->k_off, d->v_off, d->o_off},
                bss[4] = {d->q_bstride, d->k_bstride, d->v_bstride, d->o_bstride};
  const int heads[4] = {d->H, d->H / group, d->H / group, d->H};
  const char* nm[4] = {"q", "k", "v", "o"};
  for (int i = 0; i < 4; i++) {
    if (lds[i] % 4 || offs[i] % 4 || bss[i] % 4 || lds[i] < 0 || offs[i] < 0 || bss[i] < 0)
      return fail(c, ANIMA_E_ARG, "anima_attention: %s ld/off/bstride must be non-negative multiples of 4", nm[i]);
    if (lds[i] < offs[i] + (int64_t)heads[i] * d->D)
      return fail(c, ANIMA_E_ARG, "anima_attention: %s rows of %lld elements cannot hold off %lld + %d heads x %d", nm[i],
                  (long long)lds[i], (long long)offs[i], heads[i], d->D);
  }
  if (!al16(d->q) || !al16(d->k) || !al16(d->v) || !al16(d->o))
    return fail(c, ANIMA_E_ARG, "anima_attention: q/k/v/o must be 16-byte aligned");
  return ANIMA_OK;
}

// Key ranges of the chunked P.V product: 1 unless its grid has fewer than 1024 tiles; then up to
// 8 ranges of at least 1024 keys, each a multiple of the 32-key k-tile (so a range never reads past
// the valid keys).
static int pv_splits(int rows, int D, int valid) {
  const int64_t tiles = (int64_t)((rows + TG_BM - 1) / TG_BM) * ((D + TG_BN - 1) / TG_BN);
  int ks = 1;
  while (ks < 8 && tiles * ks < 1024 && valid % (2 * ks * TG_BK) == 0 && valid / (2 * ks) >= 1024) ks *= 2;
  return ks;
}

// o[m][d] = (sum over the key ranges of part[z][m][d]) * rl[m]
__global__ __launch_bounds__(256) void pv_sum_kernel(const float* part, int ks, int rows, int D, const float* rl, float* o,
                                                     int64_t ldo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = (int64_t)rows * D;
  if (i >= n) return;
  float acc = part[i];
  for (int z = 1; z < ks; z++) acc = acc + part[(int64_t)z * n + i];
  const int64_t m = i / D;
  o[m * ldo + (i - m * D)] = acc * rl[m];
}

int attention_chunked_launch(anima_ctx* c, const anima_attn_desc* d, const int* kv_len) {
  const int group = d->group <= 0 ? 1 : d->group;
  const int D = d->D, Lq = d->Lq, Lk = d->Lk;
  const float scale = d->scale != 0.0f ? d->scale : 1.0f / sqrtf((float)D);
  const bool split = d->precision == ANIMA_PREC_FP32;
  // score rows per chunk: at most 1 GiB of scores (one chunk for the VAE's 16384 tokens at 1024x1024;
  // the device has 288 GB), a multiple of the 128-row tile
  int64_t rows = std::max<int64_t>(TG_BM, ((int64_t)(1 << 30) / 4 / Lk) / TG_BM * TG_BM);
  rows = std::min<int64_t>(rows, ((int64_t)Lq + TG_BM - 1) / TG_BM * TG_BM);
  const int64_t ldk4 = ((int64_t)Lk + 3) / 4 * 4;  // row stride of the scores and of V^T (16-byte rows)
  const size_t s_bytes = (size_t)rows * ldk4 * 4, l_bytes = ((size_t)rows * 4 + 255) / 256 * 256,
               vt_bytes = ((size_t)D * ldk4 * 4 + 255) / 256 * 256;
  int max_ks = 1;
  for (int b = 0; b < d->B; b++) max_ks = std::max(max_ks, pv_splits((int)rows, D, kv_len[b]));
  const size_t p_bytes = max_ks > 1 ? (size_t)max_ks * rows * D * 4 : 0;
  void* ws = nullptr;
  int rc = workspace(c, s_bytes + l_bytes + vt_bytes + p_bytes, &ws);
  if (rc) return rc;
  float* S = (float*)ws;
  float* L = (float*)((char*)ws + s_bytes);
  float* VT = (float*)((char*)ws + s_bytes + l_bytes);
  float* P = (float*)((char*)ws + s_bytes + l_bytes + vt_bytes);
  for (int b = 0; b < d->B; b++) {
    const int valid = kv_len[b];
    for (int h = 0; h < d->H; h++) {
      const int hk = h / group;
      if (h % group == 0) {  // V^T of this kv head
        const float* v = d->v + (int64_t)b * d->v_bstride + d->v_off + (int64_t)hk * D;
        Launch lt(c, "attn.chunk.transpose_v", 0.0, 8.0 * Lk * D);
        hipLaunchKernelGGL(transpose_kernel, dim3((Lk + 31) / 32, (D + 31) / 32), dim3(256), 0, c->stream, v, d->ldv, Lk, D,
                           VT, ldk4);
        if ((rc = lt.end())) return rc;
      }
      for (int r0 = 0; r0 < Lq; r0 += (int)rows) {
        const int nr = (int)std::min<int64_t>(rows, Lq - r0);
        TGemmArgs qk{};
        qk.a = d->q + (int64_t)b * d->q_bstride + (int64_t)r0 * d->ldq + d->q_off + (int64_t)h * D;
        qk.lda = d->ldq;
        qk.b = d->k + (int64_t)b * d->k_bstride + d->k_off + (int64_t)hk * D;
        qk.ldb = d->ldk;
        qk.c = S;
        qk.ldc = ldk4;
        qk.alpha = 1.0f;
        qk.M = nr;
        qk.N = Lk;
        qk.K = D;
        if ((rc = tgemm_launch(c, qk, TG_A_ROWS, TG_B_F32, split, 1, "attn.chunk.qk", 2.0 * nr * Lk * D))) return rc;
        {
          Launch ls(c, "attn.chunk.softmax", 0.0, 8.0 * nr * Lk);
          const int cz = d->causal ? 1 : 0;
          if (Lk <= 256 * 16)
            hipLaunchKernelGGL(chunk_softmax_reg_kernel<16>, dim3(nr), dim3(256), 0, c->stream, S, ldk4, L, Lk, valid, scale, r0, cz);
          else if (Lk <= 256 * 32)
            hipLaunchKernelGGL(chunk_softmax_reg_kernel<32>, dim3(nr), dim3(256), 0, c->stream, S, ldk4, L, Lk, valid, scale, r0, cz);
          else if (Lk <= 256 * 64)
            hipLaunchKernelGGL(chunk_softmax_reg_kernel<64>, dim3(nr), dim3(256), 0, c->stream, S, ldk4, L, Lk, valid, scale, r0, cz);
          else
            hipLaunchKernelGGL(chunk_softmax_kernel, dim3(nr), dim3(256), 0, c->stream, S, ldk4, L, Lk, valid, scale, r0, cz);
          if ((rc = ls.end())) return rc;
        }
        TGemmArgs pv{};
        pv.a = S;
        pv.lda = ldk4;
        pv.b = VT;
        pv.ldb = ldk4;
        pv.alpha = 1.0f;
        pv.M = nr;
        pv.N = D;
        float* o = d->o + (int64_t)b * d->o_bstride + (int64_t)r0 * d->ldo + d->o_off + (int64_t)h * D;
        // A grid of few tiles over a long key range (the VAE's 16384 keys x 384 dims: 384 tiles)
        // splits the keys into ks ranges, products into ks partial outputs, summed and scaled by
        // 1 / rowsum afterwards
        const int ks = pv_splits(nr, D, valid);
        if (ks > 1) {
          pv.c = P;
          pv.ldc = D;
          pv.c_bs = (int64_t)nr * D;
          pv.a_bs = valid / ks;
          pv.b_bs = valid / ks;
          pv.K = valid / ks;
          if ((rc = tgemm_launch(c, pv, TG_A_ROWS, TG_B_F32, split, ks, "attn.chunk.pv", 2.0 * nr * valid * D))) return rc;
          Launch lsum(c, "attn.chunk.pv_sum", 0.0, 4.0 * nr * D * (ks + 1));
          const int64_t n = (int64_t)nr * D;
          hipLaunchKernelGGL(pv_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, c->stream, P, ks, nr, D, L, o,
                             d->ldo);
          if ((rc = lsum.end())) return rc;
        } else {
          pv.c = o;
          pv.ldc = d->ldo;
          pv.rs = L;
          pv.K = valid;  // columns past the valid keys hold zero weights
          if ((rc = tgemm_launch(c, pv, TG_A_ROWS, TG_B_F32, split, 1, "attn.chunk.pv", 2.0 * nr * valid * D))) return rc;
        }
      }
    }
  }
  return ANIMA_OK;
}

}  // namespace anima
