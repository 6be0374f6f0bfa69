// Quantized linears for gfx950: ops.linear -> matmulShader (app/gpu/gemm.js:166-280) with the
// i8 / w4 B-loaders (gemm.js:129-159), re-designed as W8A8 on the int8 matrix cores.
//
//   gemm_i8   C = epi((qx @ qw^T) * s_x[m] * s_w[n]) with v_mfma_i32_32x32x32_i8 (exact int32
//             accumulation).  Block tile 128x128, k-tile 64, 4 waves of 64x64, double-buffered
//             LDS with 80-byte rows (conflict-free 16-byte fragment reads).
//             W4: the weight tile is decoded in the loader, nibble -> int8 grid value through a
//             16-entry table per 16-weight group.  The table of a group depends only on its fp8
//             s_rel byte, so each workgroup first builds all 256 possible tables,
//             T[s][c] = clamp(rint(codebook[c] * fp8(s)), -127, 127) (tools/quant.py:127-129),
//             in LDS; decoding is then one 16-byte LDS read per group plus byte permutes.
//   gemm_f32w bf16 weights (x_embedder, final layer, timestep / adaLN projections): fp32 FMA
//             with fp32 activations, the reference's own arithmetic (gemm.js:108-128).
#include <cmath>

#include "common.h"
#include "internal.h"

namespace anima {

struct GemmArgs {
  const int8_t* qx;   // [M][K]
  const float* sx;    // [M]
  const void* w;      // i8 [N][K] | w4 codes [N][K/2]
  const float* sw;    // [N]
  const uint8_t* srel;
  const float* cb;
  const float* bias;
  float* out;
  int64_t ldc;
  float alpha;
  int act, epi;
  const float* gate;
  int64_t gate_off;
  int32_t* acc_out;
  int M, N, K;
  const float* add;  // optional [M][ld_add] term after the bias
  int64_t ld_add;
  // Attention operand epilogue of the stacked QKV projection (gemm_i8_256<STORE, W4, true>):
  // columns [kcol, vcol) are K and [vcol, N) V, H heads of 128 each; they leave as the attention's
  // bf16 K rows [B][H][Lkp][128] (RMSNorm + RoPE applied) and V^T rows [B][H][128][Lkp] (keys in
  // the MFMA order) in kv instead of out, which receives only the Q columns [0, kcol).
  void* kv;
  int64_t kv_plane;  // bytes of the K plane (the V^T plane follows)
  const float* kn;   // [128] k RMSNorm weight
  const float* cs;   // RoPE table: cos [rows][64], sin at + sin_off
  int64_t sin_off;
  float eps;
  int L, Lkp, H;     // tokens per batch element (M = B * L, L % 64 == 0 so Lkp = L), heads
  int kcol, vcol;
  // LoRA B product in the epilogue (gemm_i8_256<..., LORA>): y += sum_k lx[m][k] * B[n][k], k < lr,
  // with B as three bf16 planes lb [3][N][lr] (the scales folded in); lr % 16 == 0.  lcols > 0
  // (a multiple of 256, so a tile lies in one block): columns of block n / lcols read lx columns
  // (n / lcols) * lr + k
  const float* lx = nullptr;
  int64_t ld_lx = 0;
  const uint16_t* lb = nullptr;
  int lr = 0;
  int lcols = 0;
  // prepared Q of the QKV / Q-only projection (kv_epi_k<true>): q_norm weights (or null), the
  // bf16 [M][H][128] destination, the attention's scale * log2(e), RoPE on Q or not
  const float* qn = nullptr;
  uint16_t* qp = nullptr;
  float qc = 0.0f;
  int qrope = 0;
};


// three bf16 pieces of 8 fp32 values, two at a time (packed round-to-nearest-even conversions;
// bf16 -> fp32 is exact, so each remainder is exact)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split3_pair(f32x2_t v, bf16x2_t& h, bf16x2_t& m, bf16x2_t& l) {
  h = __builtin_convertvector(v, bf16x2_t);
  const f32x2_t r = v - __builtin_convertvector(h, f32x2_t);
  m = __builtin_convertvector(r, bf16x2_t);
  l = __builtin_convertvector(r - __builtin_convertvector(m, f32x2_t), bf16x2_t);
}
__device__ __forceinline__ void split3(float4 a, float4 b, bf16x8 (&o)[3]) {
  bf16x2_t h0, m0, l0, h1, m1, l1, h2, m2, l2, h3, m3, l3;
  split3_pair(f32x2_t{a.x, a.y}, h0, m0, l0);
  split3_pair(f32x2_t{a.z, a.w}, h1, m1, l1);
  split3_pair(f32x2_t{b.x, b.y}, h2, m2, l2);
  split3_pair(f32x2_t{b.z, b.w}, h3, m3, l3);
  o[0] = bf16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
  o[1] = bf16x8{m0[0], m0[1], m1[0], m1[1], m2[0], m2[1], m3[0], m3[1]};
  o[2] = bf16x8{l0[0], l0[1], l1[0], l1[1], l2[0], l2[1], l3[0], l3[1]};
}

// acc += sum_{i+j<=2} a_i b_j, smallest terms first
__device__ __forceinline__ f32x16 mfma_s3(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x16 acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld_bf8(const uint16_t* p) {
  const uint4 u = *(const uint4*)p;
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

__device__ __forceinline__ float apply_act(float r, int act) {
  if (act == ANIMA_ACT_GELU) return gelu_erf(r);
  if (act == ANIMA_ACT_SILU) return silu_f(r);
  return r;
}

__device__ __forceinline__ void epilogue_store(const GemmArgs& a, int m, int n, float r) {
  if (a.bias) r = r + a.bias[n];
  if (a.add) r = r + a.add[(int64_t)m * a.ld_add + n];
  r = apply_act(r, a.act);
  float* c = a.out + (int64_t)m * a.ldc + n;
  if (a.epi == ANIMA_EPI_STORE) *c = r;
  else if (a.epi == ANIMA_EPI_RESID) *c = *c + r;
  else *c = __builtin_fmaf(a.gate[a.gate_off + n], r, *c);
}

__device__ __forceinline__ float fp8e4m3(uint32_t b) {  // app/gpu/gemm.js:144-151
  const uint32_t e = (b >> 3) & 15u;
  const float m = (float)(b & 7u);
  float v = e == 0 ? m * 0.001953125f : (1.0f + m * 0.125f) * __builtin_ldexpf(1.0f, (int)e - 7);
  return (b & 128u) ? -v : v;
}

// 4 nibbles -> 4 table bytes (table = 16 bytes in t0..t3).  x holds the nibbles' bit 3 as the
// sign bit of each byte (bits 0..2 of the selector bytes in sel).  Entries 0..7 and 8..15 come
// from two byte permutes; the choice between them is a byte mask made from the four sign bits
// by a third permute (selectors 8..11 replicate the sign of bytes 1, 3, 5, 7 of {x << 8, x}).
__device__ __forceinline__ uint32_t lut4(uint32_t sel, uint32_t x, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);  // entries 0..7
  const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);  // entries 8..15
  const uint32_t mask = __builtin_amdgcn_perm(x << 8, x, 0x090b080au);
  return (hi & mask) | (lo & ~mask);
}
// even nibbles (low, k = 0, 2, 4, 6) and odd nibbles (high, k = 1, 3, 5, 7) of a code word
__device__ __forceinline__ uint32_t lut4_even(uint32_t w, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  return lut4(w & 0x07070707u, w << 4, t0, t1, t2, t3);
}
__device__ __forceinline__ uint32_t lut4_odd(uint32_t w, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  return lut4((w >> 4) & 0x07070707u, w, t0, t1, t2, t3);
}

// 8 consecutive 4-bit codes (low nibble = even k) -> 8 int8 values in k order.
__device__ __forceinline__ uint2 decode8(uint32_t w, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t ev = lut4_even(w, t0, t1, t2, t3);  // k = 0, 2, 4, 6
  const uint32_t od = lut4_odd(w, t0, t1, t2, t3);   // k = 1, 3, 5, 7
  return make_uint2(__builtin_amdgcn_perm(od, ev, 0x05010400u), __builtin_amdgcn_perm(od, ev, 0x07030602u));
}

constexpr int GBM = 128, GBN = 128, GBK = 64, GROW = GBK + 16;  // LDS row stride 80 B

template <bool W4>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t As[2][GBM * GROW];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][GBN * GROW];
  __shared__ __attribute__((aligned(16))) uint32_t lut[W4 ? 256 * 4 : 1];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, hf = lane >> 5;
  const int bm = blockIdx.y * GBM, bn = blockIdx.x * GBN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

  if constexpr (W4) {
    for (int i = tid; i < 256 * 4; i += 256) {
      const int sb = i >> 2, q = i & 3;
      const float s = fp8e4m3((uint32_t)sb);
      uint32_t packed = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float v = rintf(a.cb[4 * q + j] * s);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        packed |= ((uint32_t)(int32_t)v & 0xffu) << (8 * j);
      }
      lut[i] = packed;
    }
  }

  // loader assignment: row tid/2, 32 k at (tid&1)*32
  const int lr = tid >> 1, lk = (tid & 1) * 32;
  const bool arow = bm + lr < a.M, brow = bn + lr < a.N;
  const int8_t* ag = a.qx + (int64_t)(bm + lr) * a.K + lk;
  uint4 ar[2], br[2];
  uint4 bcodes;
  uint32_t bs2 = 0;
  auto gload = [&](int kt) {
    const int k0 = kt * GBK;
    if (arow) {
      ar[0] = *(const uint4*)(ag + k0);
      ar[1] = *(const uint4*)(ag + k0 + 16);
    } else {
      ar[0] = ar[1] = make_uint4(0, 0, 0, 0);
    }
    if constexpr (!W4) {
      if (brow) {
        const int8_t* bg = (const int8_t*)a.w + (int64_t)(bn + lr) * a.K + k0 + lk;
        br[0] = *(const uint4*)bg;
        br[1] = *(const uint4*)(bg + 16);
      } else {
        br[0] = br[1] = make_uint4(0, 0, 0, 0);
      }
    } else {
      if (brow) {
        const uint8_t* cg = (const uint8_t*)a.w + (int64_t)(bn + lr) * (a.K / 2) + (k0 + lk) / 2;
        bcodes = *(const uint4*)cg;
        const uint8_t* sg = a.srel + (int64_t)(bn + lr) * (a.K / 16) + (k0 + lk) / 16;
        bs2 = (uint32_t)sg[0] | ((uint32_t)sg[1] << 8);
      } else {
        bcodes = make_uint4(0, 0, 0, 0);
        bs2 = 0xffffffffu;  // marker: zero row
      }
    }
  };
  auto lstore = [&](int st) {
    uint4* ad = (uint4*)(As[st] + lr * GROW + lk);
    ad[0] = ar[0];
    ad[1] = ar[1];
    uint4* bd = (uint4*)(Bs[st] + lr * GROW + lk);
    if constexpr (!W4) {
      bd[0] = br[0];
      bd[1] = br[1];
    } else {
      if (bs2 == 0xffffffffu) {
        bd[0] = bd[1] = make_uint4(0, 0, 0, 0);
      } else {
        const uint4 t0 = *(const uint4*)&lut[4 * (bs2 & 0xffu)];
        const uint4 t1 = *(const uint4*)&lut[4 * ((bs2 >> 8) & 0xffu)];
        const uint2 d0 = decode8(bcodes.x, t0.x, t0.y, t0.z, t0.w);
        const uint2 d1 = decode8(bcodes.y, t0.x, t0.y, t0.z, t0.w);
        const uint2 d2 = decode8(bcodes.z, t1.x, t1.y, t1.z, t1.w);
        const uint2 d3 = decode8(bcodes.w, t1.x, t1.y, t1.z, t1.w);
        bd[0] = make_uint4(d0.x, d0.y, d1.x, d1.y);
        bd[1] = make_uint4(d2.x, d2.y, d3.x, d3.y);
      }
    }
  };

  i32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (i32x16){};

  const int nk = a.K / GBK;
  if (W4) __syncthreads();  // table ready
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    const int st = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      i32x4 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        af[i] = *(const i32x4*)(As[st] + (wm + 32 * i + lq) * GROW + 32 * ks + 16 * hf);
        bf[i] = *(const i32x4*)(Bs[st] + (wn + 32 * i + lq) * GROW + 32 * ks + 16 * hf);
      }
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(st ^ 1);
    __syncthreads();
  }

  // epilogue: lane (n + 32g), register r -> row 8(r/4) + 4g + r%4
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = bn + wn + 32 * j + lq;
    if (n >= a.N) continue;
    const float swn = a.sw[n];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = bm + wm + 32 * i + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (m >= a.M) continue;
        const int32_t v = acc[i][j][r];
        if (a.acc_out) a.acc_out[(int64_t)m * a.N + n] = v;
        float y = (float)v * a.sx[m];
        y = y * swn;
        if (a.alpha != 1.0f) y = y * a.alpha;
        epilogue_store(a, m, n, y);
      }
  }
}

// ------------------------------------------------------------------ 256x256 epilogue
//
// The 256x256 kernel multiplies with the weight fragment as srcA, so each 32x32 accumulator
// tile is C^T: for lane (l, g) register r holds row m = (tile row) + l and column
// n + 8(r/4) + r%4 with n = (tile column) + 4g.  Four consecutive columns of one row sit in four
// consecutive registers and move as one 16-byte access; the row scale is one value per lane.
// Arithmetic order is that of epilogue_store.
struct EpiCols {  // per-column scales of one 32-column tile for this lane: columns n + 8q + e
  f32x4 sw[4];    // (a bias, rare, and the gate are read where they are used)
};

__device__ __forceinline__ void epi_cols(const GemmArgs& a, int n, EpiCols& c) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const bool ok = n + 8 * q < a.N;  // N % 4 == 0: a 4-column group is all in or all out
    const int nq = ok ? n + 8 * q : 0;
    c.sw[q] = *(const f32x4*)(a.sw + nq);
  }
}

// residual C of one tile (RESID / GATED), rows past M and columns past N read as zero
__device__ __forceinline__ void epi_load_c(const GemmArgs& a, int m, int n, f32x4 (&cv)[4]) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const bool ok = m < a.M && n + 8 * q < a.N;
    cv[q] = ok ? *(const f32x4*)(a.out + (int64_t)m * a.ldc + n + 8 * q) : (f32x4){};
  }
}

// The plain epilogues with the LoRA B product (gemm_i8_256<..., LORA>), for the wave's 4 x 2
// tiles of 32 x 32 in the C^T layout, in three phases: (1) every accumulator becomes its fp32
// y = (acc * s_x) * s_w (* alpha) (+ bias) in place; (2) per 16-k slice of the rank, the slice's
// operands of all eight tiles are loaded at once -- the B planes of the two column groups (A
// operand: lane lq holds row n + lq) and the activations of the four row groups (B operand: lane
// lq holds row m, split into three bf16 terms in registers) -- and six v_mfma_f32_32x32x16_bf16
// per tile (mfma_s3) add sum_k lx[m][k] * B[n][k] onto y, so that one load latency per slice is
// exposed, not one per tile; (3) activation and store / residual / gate as in epi_store_t.
// Every lane takes part in the MFMAs (rows past M and columns past N read zeros).
template <int BSTEP>
__device__ __forceinline__ void lora_y(const GemmArgs& a, const i32x16 (&acc)[4][2], int m0, int n0, int hf, int lq,
                                       const float (&sxv)[4], f32x16 (&y)[4][2]) {
  if (a.acc_out) {  // the raw accumulators first: acc is dead once y is formed
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int m = m0 + 32 * i, nq = n0 + BSTEP * j + 8 * q;
          if (m < a.M && nq < a.N)
#pragma unroll
            for (int e = 0; e < 4; e++) a.acc_out[(int64_t)m * a.N + nq + e] = acc[i][j][4 * q + e];
        }
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    EpiCols c;
    epi_cols(a, n0 + BSTEP * j, c);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int nq = n0 + BSTEP * j + 8 * q;
      const bool ok = nq < a.N;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float b = a.bias && ok ? a.bias[nq + e] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float t = (float)acc[i][j][4 * q + e] * sxv[i];
          t = t * c.sw[q][e];
          if (a.alpha != 1.0f) t = t * a.alpha;
          if (a.bias) t = t + b;
          y[i][j][4 * q + e] = t;
        }
      }
    }
  }
  const int64_t plane = (int64_t)a.N * a.lr;
  const bf16x8 z8 = {};
  const float4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
  // the tile's rank block (wave-uniform; taken to a scalar register, which keeps the division's
  // vector temporaries from raising the kernel's register pressure into main-loop spills)
  const float* lx = a.lx + (int64_t)__builtin_amdgcn_readfirstlane(a.lcols ? (n0 / a.lcols) * a.lr : 0);
  for (int k0 = 0; k0 < a.lr; k0 += 16) {
    bf16x8 bv[2][3];
    float4 xr[4][2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int nr = n0 - 4 * hf + BSTEP * j + lq;
      const bool nok = nr < a.N;
      const uint16_t* bp = a.lb + (int64_t)(nok ? nr : 0) * a.lr + 8 * hf + k0;
#pragma unroll
      for (int p = 0; p < 3; p++) bv[j][p] = nok ? ld_bf8(bp + p * plane) : z8;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = m0 + 32 * i;
      const bool mok = m < a.M;
      const float* xp = lx + (int64_t)(mok ? m : 0) * a.ld_lx + 8 * hf + k0;
      xr[i][0] = mok ? *(const float4*)xp : z4;
      xr[i][1] = mok ? *(const float4*)(xp + 4) : z4;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      bf16x8 xv[3];
      split3(xr[i][0], xr[i][1], xv);
#pragma unroll
      for (int j = 0; j < 2; j++) y[i][j] = mfma_s3(bv[j], xv, y[i][j]);
    }
  }
}

// Phase (3) of the LoRA epilogue: activation and store / residual / gate of y.
template <int EPI, int BSTEP>
__device__ __forceinline__ void lora_store(const GemmArgs& a, const f32x16 (&y)[4][2], int m0, int n0) {
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // one tile at a time: keeps the residual loads from being hoisted above the earlier tiles'
      // stores (32 residual quads in flight would not fit beside the 128 registers of y)
      __builtin_amdgcn_sched_barrier(0);
      const int m = m0 + 32 * i;
      if (m >= a.M) continue;
      float* orow = a.out + (int64_t)m * a.ldc;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int nq = n0 + BSTEP * j + 8 * q;
        if (nq >= a.N) continue;
        f32x4 yq = {y[i][j][4 * q], y[i][j][4 * q + 1], y[i][j][4 * q + 2], y[i][j][4 * q + 3]};
        if (a.act == ANIMA_ACT_GELU) {
#pragma unroll
          for (int e = 0; e < 4; e++) yq[e] = gelu_erf(yq[e]);
        } else if (a.act == ANIMA_ACT_SILU) {
#pragma unroll
          for (int e = 0; e < 4; e++) yq[e] = silu_f(yq[e]);
        }
        f32x4 o;
        if constexpr (EPI == ANIMA_EPI_STORE) {
          o = yq;
        } else {
          const f32x4 cq = *(const f32x4*)(orow + nq);
          if constexpr (EPI == ANIMA_EPI_RESID) {
            o = cq + yq;
          } else {
            const f32x4 gt = *(const f32x4*)(a.gate + a.gate_off + nq);
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = __builtin_fmaf(gt[e], yq[e], cq[e]);
          }
        }
        *(f32x4*)(orow + nq) = o;
      }
    }
}

template <int EPI>
__device__ __forceinline__ void lora_epilogue(const GemmArgs& a, const i32x16 (&acc)[4][2], int m0, int n0, int hf,
                                              int lq, const float (&sxv)[4]) {
  f32x16 y[4][2];
  lora_y<32>(a, acc, m0, n0, hf, lq, sxv, y);
  lora_store<EPI, 32>(a, y, m0, n0);
}

template <int EPI>
__device__ __forceinline__ void epi_store_t(const GemmArgs& a, const i32x16& v, int m, int n, float sx,
                                            const EpiCols& c, const f32x4 (&cv)[4]) {
  if (m >= a.M) return;
  float* orow = a.out + (int64_t)m * a.ldc;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int nq = n + 8 * q;
    if (nq >= a.N) continue;
    if (a.acc_out) {
#pragma unroll
      for (int e = 0; e < 4; e++) a.acc_out[(int64_t)m * a.N + nq + e] = v[4 * q + e];
    }
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float t = (float)v[4 * q + e] * sx;
      y[e] = t * c.sw[q][e];
    }
    if (a.alpha != 1.0f) y = y * a.alpha;
    if (a.bias) y = y + *(const f32x4*)(a.bias + nq);
    if (a.add) y = y + *(const f32x4*)(a.add + (int64_t)m * a.ld_add + nq);
    if (a.act == ANIMA_ACT_GELU) {
#pragma unroll
      for (int e = 0; e < 4; e++) y[e] = gelu_erf(y[e]);
    } else if (a.act == ANIMA_ACT_SILU) {
#pragma unroll
      for (int e = 0; e < 4; e++) y[e] = silu_f(y[e]);
    }
    f32x4 o;
    if constexpr (EPI == ANIMA_EPI_STORE) {
      o = y;
    } else if constexpr (EPI == ANIMA_EPI_RESID) {
      o = cv[q] + y;
    } else {
      const f32x4 gt = *(const f32x4*)(a.gate + a.gate_off + nq);
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = __builtin_fmaf(gt[e], y[e], cv[q][e]);
    }
    *(f32x4*)(orow + nq) = o;
  }
}

// ------------------------------------------------------------------ attention operand epilogue
constexpr int HD_K = 128;  // head dim of the attention operands
//
// The stacked QKV projection of a DiT block can hand its K and V columns to the attention in the
// operand layout that anima_attention_prepare_kv writes (what attn_prep_kv_lines computes from the
// fp32 output), bit for bit: y is the store epilogue's fp32 value; K rows get
// x = (y * rn) * w, rn = 1 / sqrt(fma(ss, 1/128, eps)), then the split-half RoPE
// lo' = fma(lo, c, -(hi * s)), hi' = fma(hi, c, lo * s), rounded to bf16; V goes to V^T rows
// rounded to bf16.  The row sum of squares ss of a head's 128 columns uses one fixed tree:
// leaves of 8 values (columns 8q' + e and 64 + 8q' + e, e = 0..3: fmaf of the squares in that
// order), pairs of leaves q' = 2t, 2t + 1 (t = 0, 1 within a 32-column group and half), then the
// two 4-column halves, then the two 32-column groups of each 64 (the prep kernel's lane
// butterfly reaches the same sums: fp addition is commutative).

// K tile: lane (lq, hf) of wave w holds rows m0 + 32i and columns n0 + 8q + e (j = 0) and
// n0 + 64 + 8q + e (j = 1) of head (col0 - kcol) / 128 + w / 4; waves w and w ^ 2 hold the other
// 64 columns of the same rows and exchange one partial sum per row through LDS.
__device__ __forceinline__ f32x4 kv_epi_y(const GemmArgs& a, const i32x16& v, int q, float sx, int n) {
  // the store epilogue's fp32 value of columns n + 8q .. n + 8q + 3 (epi_store_t's order; the
  // QKV tiles are whole, so every column group is in range)
  const f32x4 sw = *(const f32x4*)(a.sw + n + 8 * q);
  f32x4 y;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float t = (float)v[4 * q + e] * sx;
    y[e] = t * sw[e];
  }
  if (a.alpha != 1.0f) y = y * a.alpha;
  if (a.bias) y = y + *(const f32x4*)(a.bias + n + 8 * q);
  return y;
}

// yf(i, j, q): the fp32 store values of row group i, column group j (+ 64 j), quad q.
// Q (the prepared-Q form of the attention) goes through the same steps: its own weights (none:
// no RMSNorm), RoPE when a.qrope, then times a.qc (the attention's scale * log2(e)) before the
// bf16 rounding, into row-major [M][H][128].
template <bool Q, class YF>
__device__ __forceinline__ void kv_epi_k(const GemmArgs& a, const YF& yf, int m0, int n0, int col0, int wave, int hf,
                                         int lq, float* xch) {
  const int grp = (wave >> 1) & 1;
  const int c0 = 32 * grp + 4 * hf;  // this lane's first column within the head (< 64)
  const int head = (col0 - (Q ? 0 : a.kcol)) / HD_K + (wave >> 2);
  const float* wn = Q ? a.qn : a.kn;
  const bool norm = !Q || wn, rope = !Q || a.qrope;  // (uniform over the workgroup)
  // One 32-row block at a time: the partial sum of squares over this lane pair's 64 columns goes
  // to LDS, a barrier, the partner wave's partial completes the row, and the block's values are
  // recomputed (the same fp32 bits), normalized, rotated, rounded and stored.  (One barrier for all
  // four blocks keeps the first pass's values alive into the second: the spills cost more.)
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float rn = 1.0f;
    if (norm) {
      float lf[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const f32x4 y = yf(i, j, q);
#pragma unroll
          for (int e = 0; e < 4; e++) lf[q] = __builtin_fmaf(y[e], y[e], lf[q]);
        }
      float part = (lf[0] + lf[1]) + (lf[2] + lf[3]);
      part = part + __shfl_xor(part, 32);
      if (hf == 0) xch[wave * 128 + 32 * i + lq] = part;
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the partial sums are in LDS
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const float other = xch[(wave ^ 2) * 128 + 32 * i + lq];
      const float ss = grp == 0 ? part + other : other + part;
      rn = 1.0f / sqrtf(__builtin_fmaf(ss, 1.0f / 128.0f, a.eps));
    }
    const int m = m0 + 32 * i;
    if (m >= a.M) continue;
    const int b = m / a.L, l = m - b * a.L;
    const float* crow = a.cs + (int64_t)l * (HD_K / 2) + c0;
    bf16* dst = Q ? (bf16*)a.qp + ((int64_t)m * a.H + head) * HD_K + c0
                  : (bf16*)a.kv + (((int64_t)b * a.H + head) * a.Lkp + l) * HD_K + c0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const f32x4 y0 = yf(i, 0, q), y1 = yf(i, 1, q);
      f32x4 x1 = y0, x2 = y1;
      if (norm) {
        const f32x4 w0 = *(const f32x4*)(wn + c0 + 8 * q), w1 = *(const f32x4*)(wn + c0 + 64 + 8 * q);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          x1[e] = (y0[e] * rn) * w0[e];
          x2[e] = (y1[e] * rn) * w1[e];
        }
      }
      f32x4 r1 = x1, r2 = x2;
      if (rope) {
        const f32x4 cv = *(const f32x4*)(crow + 8 * q), sv = *(const f32x4*)(crow + a.sin_off + 8 * q);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          r1[e] = __builtin_fmaf(x1[e], cv[e], -(x2[e] * sv[e]));
          r2[e] = __builtin_fmaf(x2[e], cv[e], x1[e] * sv[e]);
        }
      }
      if (Q) {
        r1 = r1 * a.qc;
        r2 = r2 * a.qc;
      }
      bf16x4 lo, hi;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        lo[e] = (bf16)r1[e];
        hi[e] = (bf16)r2[e];
      }
      *(bf16x4*)(dst + 8 * q) = lo;
      *(bf16x4*)(dst + 64 + 8 * q) = hi;
    }
  }
}

// V tile: the lane's values are one token (row) x 16 columns; V^T rows are token-contiguous, so
// each pair of lanes lq, lq ^ 1 (tokens 2t, 2t + 1: adjacent in the key order too) trades
// columns and stores 4-byte token pairs, the even lane those of columns e = 0, 1, the odd lane
// e = 2, 3.  Key order of V^T within each 16-key group: keys 0-3, 8-11, 4-7, 12-15.
template <class YF>
__device__ __forceinline__ void kv_epi_v(const GemmArgs& a, const YF& yf, int m0, int n0, int col0, int wave, int hf,
                                         int lq) {
  const int c0 = 32 * ((wave >> 1) & 1) + 4 * hf;
  const int head = (col0 - a.vcol) / HD_K + (wave >> 2);
  const bool odd = lq & 1;
  bf16* vt = (bf16*)((char*)a.kv + a.kv_plane);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = m0 + 32 * i;
    const int mp = m - (odd ? 1 : 0);  // the pair's even token
    const int b = mp / a.L, l = mp - b * a.L;
    const int g16 = l & 15, pos = (l & ~15) + 4 * (((g16 >> 2) & 1) << 1 | (g16 >> 3)) + (g16 & 3);
#pragma unroll
    for (int j = 0; j < 2; j++) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const f32x4 y = yf(i, j, q);
        // own bf16 pairs: columns (e0, e1) and (e2, e3)
        const uint32_t p01 = (uint32_t)__builtin_bit_cast(uint16_t, (bf16)y[0]) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)y[1]) << 16);
        const uint32_t p23 = (uint32_t)__builtin_bit_cast(uint16_t, (bf16)y[2]) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)y[3]) << 16);
        // the even lane sends (e2, e3) and keeps (e0, e1); the odd lane the other way round
        const uint32_t send = odd ? p01 : p23, keep = odd ? p23 : p01;
        const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xb1, 0xf, 0xf, false);  // lane ^ 1
        // token pair words (even token in the low half) for the lane's two columns
        const uint32_t lo_t = odd ? got : keep, hi_t = odd ? keep : got;
        const uint32_t w0 = __builtin_amdgcn_perm(hi_t, lo_t, 0x05040100u);  // column ea: tokens (2t, 2t+1)
        const uint32_t w1 = __builtin_amdgcn_perm(hi_t, lo_t, 0x07060302u);  // column eb
        if (m < a.M) {
          const int d = c0 + 64 * j + 8 * q + (odd ? 2 : 0);
          bf16* r0 = vt + (((int64_t)b * a.H + head) * HD_K + d) * a.Lkp + pos;
          *(uint32_t*)r0 = w0;
          *(uint32_t*)(r0 + a.Lkp) = w1;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ 256x256 int8 kernel
//
// gemm_i8_256: persistent workgroups (one per CU), each walking a list of 256 x 256 output
// tiles as one stream of k stages, so the next tile's first copies are in flight while the
// current tile's epilogue runs.  8 waves (two per SIMD); wave w owns
// rows (w%2)*128 .. +128 and columns (w/2)*64 .. +64 (4 x 2 MFMA tiles, 128 accumulator
// registers).  K advances in stages of 64 bytes; four LDS stages (A tile + B tile, 16 KiB each)
// are filled three stages ahead by buffer_load_dwordx4 ... lds straight from global memory.
// Buffer resources cover the workgroup's rows only, so rows past M (N) read as zero.
// LDS tile layout: row r (an M row of A or an N row of B) holds four 16-byte k units; unit u is
// stored at slot u ^ ((r / 4) % 4), which spreads one unit index of 16 consecutive rows over
// 16 distinct bank groups (rows 4 apart would otherwise share banks in 64-byte rows).
//
// W4 weights are unpacked in registers on their way into the B tile (gemm.js:141-158 semantics):
// a 16-byte k unit of a B row is one 16-weight group = 8 code bytes + 1 s_rel byte.  Every lane
// of all 8 waves owns two (row, unit) slots of the tile; it loads their codes and s_rel bytes
// into VGPRs one stage before the stage is published, reads the group's 16-entry int8 table
// (built in LDS at kernel start for all 256 s_rel values, T[s][c] = clamp(rint(codebook[c] *
// fp8(s)), -127, 127)), turns the 16 nibbles into 16 grid bytes with byte permutes, and writes
// them to the slot the direct copy of an int8 weight would have filled.  The MFMA stream and
// the fragment reads are the int8 kernel's.
constexpr int G2_BK = 64;               // k bytes per stage
constexpr int G2_TILE = 256 * G2_BK;    // bytes of one operand tile
constexpr int G2_ST = 2 * G2_TILE;      // stage: A tile, then B tile
constexpr int G2_NST = 4;
constexpr int G2_GM = 4;                // row tiles per group of the tile order

typedef __attribute__((address_space(3))) void lds_void_t;

// Workgroup barrier without a memory fence: LDS copies are covered by explicit vmcnt waits and
// LDS reads complete before the MFMAs that consume them issue; the empty asm statements stop
// the compiler from moving memory accesses across it.
__device__ __forceinline__ void g2_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// vmcnt(n) only (expcnt and lgkmcnt at their no-wait maxima), gfx9 s_waitcnt encoding.
#define G2_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

constexpr int G2_LUT = G2_NST * G2_ST;  // W4 table offset in LDS (256 x 16 bytes)

template <int EPI, bool W4, bool KV = false, bool LORA = false, bool QP = false>
__global__ __launch_bounds__(512, 1) void gemm_i8_256(GemmArgs a) {
  static_assert(!KV || EPI == ANIMA_EPI_STORE, "the attention operand epilogue stores");
  __shared__ __attribute__((aligned(1024))) char smem[G2_NST * G2_ST + (W4 ? 4096 : 0) + (KV ? 4096 : 0)];
  // the wave index is uniform: in a scalar register, so copy offsets derived from it stay scalar
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lq = lane & 31, hf = lane >> 5;
  const int ntn = (a.N + 255) / 256, ntm = (a.M + 255) / 256;
  const int ntiles = ntn * ntm;
  // Tile order: groups of G2_GM row tiles, column-major inside a group, so the tiles that one
  // XCD's 32 CUs run at the same time form a G2_GM x 8 block whose A rows and B columns stay in
  // that XCD's L2 (row-major order would put ~2 row tiles and ~24 column tiles in flight).
  auto tile_mn = [&](int t, int& tm, int& tn) {
    const int grp = t / (G2_GM * ntn), row0 = grp * G2_GM;
    const int gm = min(G2_GM, ntm - row0), local = t - grp * (G2_GM * ntn);
    tn = local / gm;
    tm = row0 + (local - tn * gm);
  };
  const int wm = (wave & 1) * 128, wn = (wave >> 1) * 64;
  // B column tiles of this wave: bc0 and bc0 + BSTEP.  KV: columns 128 (w / 4) + 32 ((w / 2) % 2)
  // and 64 further, so that one lane holds both columns of every RoPE pair (d, d + 64) of a head,
  // and waves w, w ^ 2 (same rows) hold the head's 128 columns between them.
  const int bc0 = KV ? 128 * (wave >> 2) + 32 * ((wave >> 1) & 1) : wn;
  constexpr int BSTEP = KV ? 64 : 32;
  const int K = a.K;
  const int nk = K / G2_BK;

  // Persistent workgroups: with one workgroup per CU (gridDim.x a multiple of 8, dispatched
  // round-robin over the XCDs), XCD x owns the contiguous tile range [x*R, (x+1)*R) and its
  // workgroups stride through it, so the tiles of one row of A stay on one L2.  Otherwise
  // workgroup b takes tiles b, b + gridDim.x, ...
  const bool xcd = (gridDim.x & 7) == 0;
  const int per = xcd ? (ntiles + 7) / 8 : ntiles;
  const int first = xcd ? (blockIdx.x & 7) * per + (blockIdx.x >> 3) : blockIdx.x;
  const int stride = xcd ? (int)(gridDim.x >> 3) : (int)gridDim.x;
  const int last = xcd ? min(ntiles, ((int)(blockIdx.x & 7) + 1) * per) : ntiles;
  const int mine = first < last ? (last - first + stride - 1) / stride : 0;
  const int total = mine * nk;  // stages of this workgroup's stream (tile-major)

  // Copies: waves 0-3 (one per SIMD; wave w shares its SIMD with wave w + 4) issue all of them, so
  // the other wave of each SIMD runs an MFMA stream free of copy and M0 set-up instructions
  // (3-4% faster than eight issuing waves).  Wave w < 4 moves the 1 KiB chunks of rows
  // 16*(2*w + c) + lane/4 and the same rows + 128 of each tile (unit permuted); rows r and r + 128
  // share the permutation.  With W4 weights every wave unpacks B bytes, and every wave also
  // copies its two A chunks (those of rows 32*(w%4) + 128*(w/4) + 16*c + lane/4).
  const int row0 = 32 * (wave & 3) + (lane >> 2), row1 = row0 + 16;
  const int loff0 = row0 * K + 16 * ((lane & 3) ^ ((row0 >> 2) & 3));
  const int loff1 = row1 * K + 16 * ((lane & 3) ^ ((row1 >> 2) & 3));
  // The copy stream runs three stages ahead of the compute: ig = next stage to copy (LDS stage
  // ig % 4), is = its k-stage within tile it; ra / rb are tile it's buffer resources, which
  // cover the tile's rows only, so rows past M (N) read as zero.  Advanced incrementally (no
  // division per stage).  Past this workgroup's last stage the resources stay those of its
  // last tile, so the copies issued there (unconditionally, to keep the wait counts the same
  // on every path) re-read that tile in bounds into LDS stages no wave reads any more.
  int ig = 0, is = 0, it = 0;
  __amdgpu_buffer_rsrc_t ra, rb, rc, rs;  // A, int8 B | W4 codes, W4 s_rel
  // W4 slots of this lane: tile rows wrow + 16 c (c = 0, 1), k unit wunit of the stage (the unit
  // whose copy lands in this lane's LDS slot; rows 16 apart share it), LDS chunk
  // (wchunk + c) * 1024 + 16 * lane.  Row c = 1 is a constant byte step away (scalar offset).
  const int wrow = 32 * (wave & 3) + 128 * (wave >> 2) + (lane >> 2), wchunk = 2 * (wave & 3) + 8 * (wave >> 2);
  const int wunit = (lane & 3) ^ ((wrow >> 2) & 3);
  const int coff = wrow * (K / 2) + 8 * wunit, soff = wrow * (K / 16) + wunit;
  // W4 codes are a second stream (stage cs of tile ct next, resources rc / rs), issued between
  // the two k-steps of each iteration into one of two register sets (stage parity): stage X's
  // codes are loaded into set X % 2 during iteration X-3 and unpacked during iteration X-2.
  int cs = 0, ct = 0;
  uint2 wcode[2][2] = {};
  uint32_t wsrel[2][2] = {};
#define G2_RSRC()                                                                                             \
  {                                                                                                           \
    int tm_, tn_;                                                                                             \
    tile_mn(first + it * stride, tm_, tn_);                                                                   \
    const int bm_ = tm_ * 256, bn_ = tn_ * 256;                                                               \
    ra = __builtin_amdgcn_make_buffer_rsrc((void*)(a.qx + (int64_t)bm_ * K), (short)0, min(256, a.M - bm_) * K, \
                                           0x00020000);                                                       \
    if constexpr (!W4) {                                                                                      \
      rb = __builtin_amdgcn_make_buffer_rsrc((void*)((const int8_t*)a.w + (int64_t)bn_ * K), (short)0,         \
                                             min(256, a.N - bn_) * K, 0x00020000);                            \
    }                                                                                                         \
  }
#define G2_RSRC_C()                                                                                           \
  {                                                                                                           \
    int tm_, tn_;                                                                                             \
    tile_mn(first + ct * stride, tm_, tn_);                                                                   \
    const int bn_ = tn_ * 256;                                                                                \
    rc = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)a.w + (int64_t)bn_ * (K / 2)), (short)0,    \
                                           min(256, a.N - bn_) * (K / 2), 0x00020000);                        \
    rs = __builtin_amdgcn_make_buffer_rsrc((void*)(a.srel + (int64_t)bn_ * (K / 16)), (short)0,                \
                                           min(256, a.N - bn_) * (K / 16), 0x00020000);                       \
  }
  // W4: this lane's codes and s_rel bytes of the next codes stage into register set SET
#define G2_ISSUE_C(SET)                                                                                       \
  {                                                                                                           \
    _Pragma("unroll") for (int c_ = 0; c_ < 2; c_++) {                                                        \
      const auto v_ = __builtin_amdgcn_raw_buffer_load_b64(rc, coff, cs * (G2_BK / 2) + c_ * 8 * K, 0);       \
      wcode[SET][c_] = make_uint2(v_[0], v_[1]);                                                              \
      wsrel[SET][c_] = __builtin_amdgcn_raw_buffer_load_b8(rs, soff, cs * (G2_BK / 16) + c_ * K, 0);         \
    }                                                                                                         \
    if (++cs == nk) {                                                                                         \
      cs = 0;                                                                                                 \
      if (++ct < mine) G2_RSRC_C();                                                                           \
    }                                                                                                         \
  }
#define G2_ISSUE()                                                                                            \
  {                                                                                                           \
    char* st_ = smem + (ig & (G2_NST - 1)) * G2_ST;                                                           \
    if constexpr (W4) {                                                                                       \
      /* every wave: its two A chunks (the same chunks as its W4 slots) */                                    \
      const int so_ = is * G2_BK + (wave >> 2) * 128 * K;                                                     \
      char* sw_ = st_ + wchunk * 1024;                                                                        \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sw_), 16, loff0, so_, 0, 0);                 \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sw_ + 1024), 16, loff1, so_, 0, 0);          \
    } else if (wave < 4) {                                                                                    \
      _Pragma("unroll") for (int h_ = 0; h_ < 2; h_++) {                                                      \
        const int so_ = is * G2_BK + h_ * 128 * K;                                                            \
        char* sw_ = st_ + (2 * wave + 8 * h_) * 1024;                                                         \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sw_), 16, loff0, so_, 0, 0);               \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sw_ + 1024), 16, loff1, so_, 0, 0);        \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(sw_ + G2_TILE), 16, loff0, so_, 0, 0);     \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(sw_ + G2_TILE + 1024), 16, loff1, so_, 0, 0); \
      }                                                                                                       \
    }                                                                                                         \
    ig++;                                                                                                     \
    if (++is == nk) {                                                                                         \
      is = 0;                                                                                                 \
      if (++it < mine) G2_RSRC();                                                                             \
    }                                                                                                         \
  }
  // W4 unpack of one stage's codes (register set SET) into the B tile of LDS stage st, in three
  // steps so the loop can spread them over its MFMAs: the two group tables (w4_tables), the
  // nibble lookups (w4_lookup, part q = slot q/4, code word (q/2)%2, even / odd nibbles q%2),
  // and the byte interleave + tile write of a slot (w4_store).  The table read and the tile
  // write are explicit LDS instructions: the compiler cannot tell them apart from the in-flight
  // direct copies into other stages and would otherwise wait for all of those first.  Ordering
  // is the barrier protocol's: the slot is free after the barrier of the iteration that writes
  // it, the tables were written before the first barrier, and every wave waits lgkmcnt(0)
  // before the barrier that publishes the slot.
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
  i32x4 wt[2];         // group tables of the two slots
  uint32_t wl[2][4];   // nibble lookups: [slot][2 * word + odd]
  auto w4_tables = [&](int set) {
    if constexpr (W4) {
      asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                   : "=&v"(wt[0]), "=&v"(wt[1])
                   : "v"(lds0 + G2_LUT + 16 * (wsrel[set][0] & 0xffu)), "v"(lds0 + G2_LUT + 16 * (wsrel[set][1] & 0xffu))
                   : "memory");
    }
  };
  auto w4_lookup = [&](int set, int q) {
    if constexpr (W4) {
      const int c_ = q >> 2, word = (q >> 1) & 1, odd = q & 1;
      const uint32_t w = word ? wcode[set][c_].y : wcode[set][c_].x;
      wl[c_][q & 3] = odd ? lut4_odd(w, wt[c_][0], wt[c_][1], wt[c_][2], wt[c_][3])
                          : lut4_even(w, wt[c_][0], wt[c_][1], wt[c_][2], wt[c_][3]);
    }
  };
  auto w4_store = [&](int st, int c_) {
    if constexpr (W4) {
      // even / odd k bytes -> k order (decode8's interleave)
      const i32x4 o = {(int)__builtin_amdgcn_perm(wl[c_][1], wl[c_][0], 0x05010400u),
                       (int)__builtin_amdgcn_perm(wl[c_][1], wl[c_][0], 0x07030602u),
                       (int)__builtin_amdgcn_perm(wl[c_][3], wl[c_][2], 0x05010400u),
                       (int)__builtin_amdgcn_perm(wl[c_][3], wl[c_][2], 0x07030602u)};
      const uint32_t dst = lds0 + (st & (G2_NST - 1)) * G2_ST + G2_TILE + (wchunk + c_) * 1024 + 16 * lane;
      asm volatile("ds_write_b128 %0, %1" ::"v"(dst), "v"(o) : "memory");
    }
  };
  auto w4_unpack = [&](int set, int st) {  // all three steps at once (prologue)
    w4_tables(set);
#pragma unroll
    for (int q = 0; q < 8; q++) w4_lookup(set, q);
    w4_store(st, 0);
    w4_store(st, 1);
  };
  // fragment lane offsets: row lq of a 32-row tile, unit 2*ks + hf (k-step ks of 32 bytes)
  int fofs[2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) fofs[ks] = lq * G2_BK + 16 * ((2 * ks + hf) ^ ((lq >> 2) & 3));

  i32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (i32x16){};

  // Stage g is published (barrier) one iteration before it is computed, so the fragment reads
  // of its first k-step run under the MFMAs of stage g-1's second k-step.
  // W4: stage g's codes are issued with its A copies (iteration g-3) and unpacked into LDS at
  // iteration g-2, after the barrier that ends all reads of the LDS stage it reuses, so the
  // barrier of iteration g-1 publishes them with the A tile.
  i32x4 af0[4], bf0[2], af1[4], bf1[2];
  if constexpr (W4) {
    // the 256 tables, 4 dwords each: table s, bytes c = clamp(rint(codebook[c] * fp8(s)), -127, 127)
    for (int i = tid; i < 256 * 4; i += 512) {
      const float sv = fp8e4m3((uint32_t)(i >> 2));
      uint32_t packed = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float v = rintf(a.cb[4 * (i & 3) + j] * sv);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        packed |= ((uint32_t)(int32_t)v & 0xffu) << (8 * j);
      }
      *(uint32_t*)(smem + G2_LUT + 4 * i) = packed;
    }
    __syncthreads();
  }
  if (total == 0) return;
  G2_RSRC();
  if constexpr (W4) {
    // stages 0 and 1 unpacked here (their copies waited for outright), stage 2 during
    // iteration 0.  From here on, per wave and iteration: 2 A copies (stage g+3, at the start),
    // then 4 code / s_rel loads (stage g+3, between the k-steps or after a tile's epilogue).
    G2_RSRC_C();
    G2_ISSUE();
    G2_ISSUE_C(0);
    G2_WAIT_VM(0);
    w4_unpack(0, 0);
    G2_ISSUE();
    G2_ISSUE_C(1);
    G2_WAIT_VM(0);
    w4_unpack(1, 1);
    G2_ISSUE();
    G2_ISSUE_C(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's unpacked B bytes are in LDS
  } else {
    if (total > 0) G2_ISSUE();
    if (total > 1) G2_ISSUE();
    if (total > 2) G2_ISSUE();
    if (total > 2) G2_WAIT_VM(16);
    else if (total > 1) G2_WAIT_VM(8);
    else G2_WAIT_VM(0);
  }
  g2_barrier();
  if (total > 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) af0[i] = *(const i32x4*)(smem + (wm + 32 * i) * G2_BK + fofs[0]);
#pragma unroll
    for (int j = 0; j < 2; j++) bf0[j] = *(const i32x4*)(smem + G2_TILE + (bc0 + BSTEP * j) * G2_BK + fofs[0]);
  }
  int s = 0, k = 0;  // stage within the tile, tile index within this workgroup's list
  // One iteration per stage g; written as a lambda over the stage parity P (a compile-time W4
  // register set), called for even and odd stages in turn.
  auto iteration = [&](const int g, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    // publish stage g+1: this wave's copies of it are done once at most those of g+2 are
    // pending; the barrier also ends every wave's reads of stage g-1, which is refilled with g+3
    if constexpr (W4) {
      // stage g+1's A copies landed (stage g+2's A copies and codes may pend: 6); this wave's
      // unpacked bytes of stage g+1 (written during iteration g-1) are in LDS
      G2_WAIT_VM(6);
      __builtin_amdgcn_s_waitcnt(0xc07f);
    } else {
      if (g + 2 < total) G2_WAIT_VM(8);
      else G2_WAIT_VM(0);
    }
    g2_barrier();
    // W4: stage g+2 is unpacked from set P during the second k-step of this iteration: its
    // tables are read between the k-steps (the only loads issued after its codes are stage
    // g+3's A copies, which stay in flight), then stage g+3's codes are issued into set 1-P.
    // Past the last stage the unpack runs on stale registers into the LDS stage of g-2, which no
    // wave reads any more (harmless, and branch-free inside the MFMA stream).  On the
    // iteration that ends a tile, stage g+3's codes are issued after the epilogue, so no code
    // registers are live across it (register pressure; one wait per tile).
    const bool late = W4 && s + 1 == nk;
    if constexpr (W4) {
      G2_ISSUE();
    } else {
      if (g + 3 < total) G2_ISSUE();
    }
    // Hand-ordered (sched_barrier fences keep the written order): each MFMA of one k-step is
    // followed by one fragment read for the next k-step, B fragments first, so a fragment is
    // read at least three MFMAs (~100 cycles) before its first use.  The second k-step reads
    // stage g+1 (unconditionally: after the last stage this reads a stale stage whose values
    // are unused; a branch here would make the compiler drain all LDS reads first).  W4, in the
    // second k-step: two nibble lookups after each of its MFMAs 1-4, one tile write after each
    // of MFMAs 5 and 6.
    const char* st = smem + (g & (G2_NST - 1)) * G2_ST;
    const char* sn = smem + ((g + 1) & (G2_NST - 1)) * G2_ST;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      acc[q >> 1][q & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf0[q & 1], af0[q >> 1], acc[q >> 1][q & 1], 0, 0, 0);
      if (q < 2) bf1[q] = *(const i32x4*)(st + G2_TILE + (bc0 + BSTEP * q) * G2_BK + fofs[1]);
      else if (q < 6) af1[q - 2] = *(const i32x4*)(st + (wm + 32 * (q - 2)) * G2_BK + fofs[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (W4) {
      w4_tables(P);
      if (!late) G2_ISSUE_C(1 - P);
    }
#pragma unroll
    for (int q = 0; q < 8; q++) {
      acc[q >> 1][q & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf1[q & 1], af1[q >> 1], acc[q >> 1][q & 1], 0, 0, 0);
      if (q < 2) bf0[q] = *(const i32x4*)(sn + G2_TILE + (bc0 + BSTEP * q) * G2_BK + fofs[0]);
      else if (q < 6) af0[q - 2] = *(const i32x4*)(sn + (wm + 32 * (q - 2)) * G2_BK + fofs[0]);
      if (q >= 1 && q <= 4) {
        w4_lookup(P, 2 * (q - 1));
        w4_lookup(P, 2 * (q - 1) + 1);
      }
      if (q == 5 || q == 6) w4_store(g + 2, q - 5);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (++s == nk && KV) {
      // tile done, attention operand epilogue: Q columns stored as fp32, K and V columns
      // converted to the attention's bf16 operand layout
      int tm, tn;
      tile_mn(first + k * stride, tm, tn);
      const int col0 = tn * 256, m0 = tm * 256 + wm + lq, n0 = col0 + bc0 + 4 * hf;
      float sxv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) sxv[i] = m0 + 32 * i < a.M ? a.sx[m0 + 32 * i] : 0.0f;
      if constexpr (LORA) {
        // y with the LoRA term (the column groups are 64 apart in this layout), then the same
        // Q store / K / V conversions on y
        f32x16 y[4][2];
        lora_y<64>(a, acc, m0, n0, hf, lq, sxv, y);
        const auto yf = [&](int i, int j, int q) {
          return f32x4{y[i][j][4 * q], y[i][j][4 * q + 1], y[i][j][4 * q + 2], y[i][j][4 * q + 3]};
        };
        float* xch = (float*)(smem + G2_NST * G2_ST + (W4 ? 4096 : 0));
        if (QP && col0 < a.kcol) kv_epi_k<true>(a, yf, m0, n0, col0, wave, hf, lq, xch);
        else if (col0 < a.kcol) lora_store<ANIMA_EPI_STORE, 64>(a, y, m0, n0);
        else if (col0 < a.vcol) kv_epi_k<false>(a, yf, m0, n0, col0, wave, hf, lq, xch);
        else kv_epi_v(a, yf, m0, n0, col0, wave, hf, lq);
      } else {
        const auto yf = [&](int i, int j, int q) { return kv_epi_y(a, acc[i][j], q, sxv[i], n0 + 64 * j); };
        float* xch = (float*)(smem + G2_NST * G2_ST + (W4 ? 4096 : 0));
        if (QP && col0 < a.kcol) {
          kv_epi_k<true>(a, yf, m0, n0, col0, wave, hf, lq, xch);
        } else if (col0 < a.kcol) {
          EpiCols cc;
          const f32x4 none[4] = {};
#pragma unroll
          for (int j = 0; j < 2; j++) {
            epi_cols(a, n0 + 64 * j, cc);
#pragma unroll
            for (int i = 0; i < 4; i++) epi_store_t<ANIMA_EPI_STORE>(a, acc[i][j], m0 + 32 * i, n0 + 64 * j, sxv[i], cc, none);
          }
        } else if (col0 < a.vcol) {
          kv_epi_k<false>(a, yf, m0, n0, col0, wave, hf, lq, xch);
        } else {
          kv_epi_v(a, yf, m0, n0, col0, wave, hf, lq);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = (i32x16){};
      s = 0;
      k++;
      if constexpr (W4) {
        if (late) G2_ISSUE_C(1 - P);
      }
    } else if (s == nk) {
      // tile done: epilogue (the next tile's first stages are already in flight), one 32x32
      // tile at a time, written out (a loop over the tiles is not fully unrolled at this size,
      // and a run-time tile index would put the accumulators in scratch memory)
      // The residual loads of the next 32x32 tile are issued before the current tile's
      // stores, so each tile's wait overlaps the previous tile's arithmetic.
      int tm, tn;
      tile_mn(first + k * stride, tm, tn);
      const int m0 = tm * 256 + wm + lq, n0 = tn * 256 + wn + 4 * hf;
      float sxv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) sxv[i] = m0 + 32 * i < a.M ? a.sx[m0 + 32 * i] : 0.0f;
      EpiCols cc;  // column operands of the current 32-column tile (reloaded for the second)
      epi_cols(a, n0, cc);
      f32x4 cA[4], cB[4];
#define G2_C(buf, i, j) \
  if constexpr (EPI != ANIMA_EPI_STORE) epi_load_c(a, m0 + 32 * (i), n0 + 32 * (j), buf);
#define G2_T(buf, i, j, cc) epi_store_t<EPI>(a, acc[i][j], m0 + 32 * (i), n0 + 32 * (j), sxv[i], cc, buf);
      if constexpr (LORA) {
        lora_epilogue<EPI>(a, acc, m0, n0, hf, lq, sxv);
      } else {
        G2_C(cA, 0, 0)
        G2_C(cB, 1, 0) G2_T(cA, 0, 0, cc)
        G2_C(cA, 2, 0) G2_T(cB, 1, 0, cc)
        G2_C(cB, 3, 0) G2_T(cA, 2, 0, cc)
        G2_C(cA, 0, 1) G2_T(cB, 3, 0, cc)
        epi_cols(a, n0 + 32, cc);
        G2_C(cB, 1, 1) G2_T(cA, 0, 1, cc)
        G2_C(cA, 2, 1) G2_T(cB, 1, 1, cc)
        G2_C(cB, 3, 1) G2_T(cA, 2, 1, cc)
        G2_T(cB, 3, 1, cc)
      }
#undef G2_C
#undef G2_T
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = (i32x16){};
      s = 0;
      k++;
      if constexpr (W4) {
        if (late) G2_ISSUE_C(1 - P);
      }
    }
  };
  for (int g = 0; g < total; g += 2) {
    iteration(g, std::integral_constant<int, 0>{});
    if (g + 1 < total) iteration(g + 1, std::integral_constant<int, 1>{});
  }
  G2_WAIT_VM(0);  // no copy into LDS outlives the workgroup
}
#undef G2_WAIT_VM
#undef G2_ISSUE
#undef G2_ISSUE_C
#undef G2_RSRC
#undef G2_RSRC_C

// ------------------------------------------------------------------ W4 -> int8 grid (load time)
//
// A W4 weight is a row-major stream of 16-weight groups: group g has code bytes [8g, 8g + 8)
// (low nibble = even k), s_rel byte g and grid bytes [16g, 16g + 16), whatever the row length
// (K % 16 == 0).  Thread = W4_UNPACK_U groups, 256 groups apart, whose loads are all issued
// before the first lookup; a wave reads 512 contiguous code bytes and 64 s_rel bytes and writes
// 1 KiB per instruction.  The 16-entry tables of all 256 s_rel values are built in LDS per
// workgroup as in the GEMMs, while the first groups' loads are in flight.
constexpr int W4_UNPACK_U = 4;
__global__ __launch_bounds__(256) void w4_unpack_kernel(const uint2* __restrict__ codes, const uint8_t* __restrict__ srel,
                                                        const float* __restrict__ cb, uint4* __restrict__ out, int64_t ngroups) {
  __shared__ __attribute__((aligned(16))) uint32_t lut[256 * 4];
  const int64_t stride = (int64_t)gridDim.x * (256 * W4_UNPACK_U);
  int64_t g0 = (int64_t)blockIdx.x * (256 * W4_UNPACK_U) + threadIdx.x;
  uint2 w[W4_UNPACK_U];
  uint32_t sr[W4_UNPACK_U];
  auto load = [&]() {
#pragma unroll
    for (int u = 0; u < W4_UNPACK_U; u++) {
      const int64_t g = g0 + 256 * u;
      if (g < ngroups) {
        w[u] = codes[g];
        sr[u] = srel[g];
      }
    }
  };
  load();
  for (int i = threadIdx.x; i < 256 * 4; i += 256) {
    const float s = fp8e4m3((uint32_t)(i >> 2));
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float v = rintf(cb[4 * (i & 3) + j] * s);
      v = fminf(fmaxf(v, -127.0f), 127.0f);
      packed |= ((uint32_t)(int32_t)v & 0xffu) << (8 * j);
    }
    lut[i] = packed;
  }
  __syncthreads();
  while (g0 < ngroups) {
#pragma unroll
    for (int u = 0; u < W4_UNPACK_U; u++) {
      const int64_t g = g0 + 256 * u;
      if (g < ngroups) {
        const uint4 t = *(const uint4*)&lut[4 * sr[u]];
        const uint2 lo = decode8(w[u].x, t.x, t.y, t.z, t.w), hi = decode8(w[u].y, t.x, t.y, t.z, t.w);
        out[g] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
    }
    g0 += stride;
    load();
  }
}

int weight_unpack_w4_launch(anima_ctx* c, const anima_weight* W, int8_t* grid);

// ANIMA_W4_GRID_SCRATCH: the int8 grid of W in a pooled buffer of N * K bytes (the caller frees
// it after the GEMM that reads it; the pool is stream-ordered), and g pointed at it as an int8
// weight.  The scale (s_channel) and bias stay the W4 weight's.
static int w4_grid_scratch(anima_ctx* c, const anima_weight* W, GemmArgs& g, void** grid) {
  *grid = nullptr;
  int rc = anima_alloc(c, (size_t)W->N * W->K, grid);
  if (rc) return rc;
  rc = weight_unpack_w4_launch(c, W, (int8_t*)*grid);
  if (rc) {
    anima_free(c, *grid);
    *grid = nullptr;
    return rc;
  }
  g.w = *grid;
  g.srel = nullptr;
  g.cb = nullptr;
  return ANIMA_OK;
}

int weight_unpack_w4_launch(anima_ctx* c, const anima_weight* W, int8_t* grid) {
  if (!W || !grid) return fail(c, ANIMA_E_ARG, "anima_weight_unpack_w4: null weight or grid");
  if (W->kind != ANIMA_W_W4) return fail(c, ANIMA_E_ARG, "anima_weight_unpack_w4: weight kind %d is not W4", W->kind);
  if (!W->w || !W->srel || !W->codebook) return fail(c, ANIMA_E_ARG, "anima_weight_unpack_w4: missing codes / s_rel / codebook");
  if (W->N < 1 || W->K < 32 || W->K % 32) return fail(c, ANIMA_E_ARG, "anima_weight_unpack_w4: N=%d K=%d (K %% 32 == 0)", W->N, W->K);
  if (((uintptr_t)W->w & 15) || ((uintptr_t)grid & 15))
    return fail(c, ANIMA_E_ARG, "anima_weight_unpack_w4: codes and grid must be 16-byte aligned");
  const int64_t ngroups = (int64_t)W->N * (W->K / 16);
  Launch L(c, "w4.unpack", 0.0, (double)W->N * W->K * 1.5 + (double)W->N * W->K / 16);
  const int64_t blocks = (ngroups + 256 * W4_UNPACK_U - 1) / (256 * W4_UNPACK_U), cap = 8LL * c->num_cus;
  hipLaunchKernelGGL(w4_unpack_kernel, dim3((unsigned)(blocks < cap ? blocks : cap)), dim3(256), 0, c->stream,
                     (const uint2*)W->w, W->srel, W->codebook, (uint4*)grid, ngroups);
  return L.end();
}

// ------------------------------------------------------------------ bf16 weights, fp32 math

struct F32WArgs {
  const float* x;
  int64_t ldx;
  const void* w;  // bf16 [N][K] (fp32 [N][K] when wf32)
  const float* bias;
  float* out;
  int64_t ldc;
  float alpha;
  int act, epi;
  const float* gate;
  int64_t gate_off;
  int M, N, K;
  // grouped GEMV only: group g = blockIdx.y reads x + g*x_gs, w + g*w_gs, bias + g*bias_gs and
  // writes out + g*out_gs (all zero for a single product)
  int64_t x_gs, w_gs, bias_gs, out_gs;
  const float* add;  // optional [M][ld_add] term after the bias
  int64_t ld_add;
  int wf32;  // fp32 weights (tile kernel only)
  int64_t ldw = 0;  // weight row stride (0: K); the split-k LDS kernel reads k-slices of longer rows
  int64_t wplane = 0;  // split weights: plane stride in elements (set by the host, N * K unless a row block)
  // split weights over per-token int8 activations (x unused): q [M][ldx] bytes, s [M] row scales,
  // y = s[m] * sum_k q[m][k] W[n][k]
  const int8_t* xq = nullptr;
  const float* xs = nullptr;
};

// 64x64 tile, 256 threads x (4x4) outputs, k-tile 16 (the small-tile layout of gemm.js:17).
__global__ __launch_bounds__(256) void gemm_f32w_kernel(F32WArgs a) {
  __shared__ float Xs[16][64 + 4];
  __shared__ float Ws[16][64 + 4];
  const int tid = threadIdx.x;
  const int bm = blockIdx.y * 64, bn = blockIdx.x * 64;
  const int tm = tid & 15, tn = tid >> 4;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < a.K; k0 += 16) {
    for (int i = tid; i < 64 * 16; i += 256) {
      const int r = i >> 4, kk = i & 15;
      const int m = bm + r, n = bn + r, k = k0 + kk;
      Xs[kk][r] = (m < a.M && k < a.K) ? a.x[(int64_t)m * a.ldx + k] : 0.0f;
      Ws[kk][r] = !(n < a.N && k < a.K) ? 0.0f
                  : a.wf32 ? ((const float*)a.w)[(int64_t)n * a.K + k]
                           : __uint_as_float((uint32_t)((const uint16_t*)a.w)[(int64_t)n * a.K + k] << 16);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float xv[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        xv[i] = Xs[kk][tm + 16 * i];
        wv[i] = Ws[kk][tn + 16 * i];
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(xv[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = bm + tm + 16 * i;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = bn + tn + 16 * j;
      if (n >= a.N) continue;
      float r = acc[i][j] * a.alpha;
      if (a.bias) r = r + a.bias[n];
      if (a.add) r = r + a.add[(int64_t)m * a.ld_add + n];
      r = apply_act(r, a.act);
      float* c = a.out + (int64_t)m * a.ldc + n;
      if (a.epi == ANIMA_EPI_STORE) *c = r;
      else if (a.epi == ANIMA_EPI_RESID) *c = *c + r;
      else *c = __builtin_fmaf(a.gate[a.gate_off + n], r, *c);
    }
  }
}

// fp32-weight linear on the fp32 matrix cores (v_mfma_f32_32x32x2_f32): the LoRA B products
// (short K = rank).  Each wave owns a 32 x 32 output tile and four waves make a 64 x 64 block; in a
// k-tile of 32, lane (l, h) holds x[row l][16h..16h+15] and W[col l][16h..16h+15] (16-byte global
// loads, no LDS) and MFMA s multiplies k = 16h + s, so the two lane halves cover the 32 k values.
// Epilogue of gemm_f32w_kernel.
__global__ __launch_bounds__(256) void gemm_f32m_kernel(F32WArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lq = lane & 31, hf = lane >> 5;
  const int m0 = blockIdx.y * 64 + (wave & 1) * 32;
  const int n0 = blockIdx.x * 64 + (wave >> 1) * 32;
  const int m = m0 + lq, n = n0 + lq;
  const bool mok = m < a.M, nok = n < a.N;
  const float* xr = a.x + (int64_t)(mok ? m : 0) * a.ldx + 16 * hf;
  const float* wr = (const float*)a.w + (int64_t)(nok ? n : 0) * a.K + 16 * hf;
  f32x16 acc = {};
  const int nkt = (a.K + 31) / 32;
  for (int kt = 0; kt < nkt; kt++) {
    const int k0 = 32 * kt;
    float xv[16], wv[16];
    if (k0 + 32 <= a.K) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 t0 = *(const float4*)(xr + k0 + 4 * j), u0 = *(const float4*)(wr + k0 + 4 * j);
        const float4 t = mok ? t0 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float4 u = nok ? u0 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        xv[4 * j] = t.x; xv[4 * j + 1] = t.y; xv[4 * j + 2] = t.z; xv[4 * j + 3] = t.w;
        wv[4 * j] = u.x; wv[4 * j + 1] = u.y; wv[4 * j + 2] = u.z; wv[4 * j + 3] = u.w;
      }
    } else {  // the last, partial k-tile
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const bool kok = k0 + 16 * hf + s < a.K;
        xv[s] = mok && kok ? xr[k0 + s] : 0.0f;
        wv[s] = nok && kok ? wr[k0 + s] : 0.0f;
      }
    }
#pragma unroll
    for (int s = 0; s < 16; s++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[s], wv[s], acc, 0, 0, 0);
  }
  if (!nok) return;
  // output layout: lane (l, h), register r -> row 8(r/4) + 4h + r%4 of the tile, column l
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int mm = m0 + 8 * (r >> 2) + 4 * hf + (r & 3);
    if (mm >= a.M) continue;
    float v = acc[r] * a.alpha;
    if (a.bias) v = v + a.bias[n];
    if (a.add) v = v + a.add[(int64_t)mm * a.ld_add + n];
    v = apply_act(v, a.act);
    float* c = a.out + (int64_t)mm * a.ldc + n;
    if (a.epi == ANIMA_EPI_STORE) *c = v;
    else if (a.epi == ANIMA_EPI_RESID) *c = *c + v;
    else *c = __builtin_fmaf(a.gate[a.gate_off + n], v, *c);
  }
}

// Weight element loads of the fp32-MFMA kernels: fp32 weights, or bf16 weights widened exactly
// (bf16 << 16) so the products and sums are those of the fp32 weights.  Four consecutive values:
// one 16-byte load (fp32) or one 8-byte load (bf16).
template <bool BF>
__device__ __forceinline__ float4 ld_w4(const void* w, int64_t i) {
  if constexpr (BF) {
    const uint2 u = *(const uint2*)((const uint16_t*)w + i);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
  } else {
    return *(const float4*)((const float*)w + i);
  }
}
template <bool BF>
__device__ __forceinline__ float ld_w1(const void* w, int64_t i) {
  if constexpr (BF) return __uint_as_float((uint32_t)((const uint16_t*)w)[i] << 16);
  else return ((const float*)w)[i];
}

// The same product with the operands swapped (W rows as MFMA A, x rows as MFMA B), so the result
// is C^T in the MFMA layout: lane (l, h) holds output row m0 + l and, in register group g, the four
// consecutive columns n0 + 8g + 4h .. + 3, which the epilogue moves as 16-byte loads / stores.
// Needs N % 4 == 0 and 16-byte aligned out / add / bias / gate rows; the LoRA B products (output
// width = model width, K = rank) are write-bound, so this is their kernel, and with bf16 weights
// (BF) that of the x_embedder (K = 68).
template <bool BF>
__global__ __launch_bounds__(256) void gemm_f32m_t_kernel(F32WArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lq = lane & 31, hf = lane >> 5;
  const int m0 = blockIdx.y * 64 + (wave & 1) * 32;
  const int n0 = blockIdx.x * 64 + (wave >> 1) * 32;
  const int m = m0 + lq, n = n0 + lq;
  const bool mok = m < a.M, nok = n < a.N;
  const float* xr = a.x + (int64_t)(mok ? m : 0) * a.ldx + 16 * hf;
  const int64_t wr = (int64_t)(nok ? n : 0) * a.K + 16 * hf;
  f32x16 acc = {};
  const int nkt = (a.K + 31) / 32;
  for (int kt = 0; kt < nkt; kt++) {
    const int k0 = 32 * kt;
    float xv[16], wv[16];
    if (k0 + 32 <= a.K) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        // unconditional in-bounds loads (rows clamped), then selects: no branch per load
        const float4 t0 = *(const float4*)(xr + k0 + 4 * j);
        const float4 u0 = ld_w4<BF>(a.w, wr + k0 + 4 * j);
        const float4 t = mok ? t0 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float4 u = nok ? u0 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        xv[4 * j] = t.x; xv[4 * j + 1] = t.y; xv[4 * j + 2] = t.z; xv[4 * j + 3] = t.w;
        wv[4 * j] = u.x; wv[4 * j + 1] = u.y; wv[4 * j + 2] = u.z; wv[4 * j + 3] = u.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const bool kok = k0 + 16 * hf + s < a.K;
        xv[s] = mok && kok ? xr[k0 + s] : 0.0f;
        wv[s] = nok && kok ? ld_w1<BF>(a.w, wr + k0 + s) : 0.0f;
      }
    }
#pragma unroll
    for (int s = 0; s < 16; s++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[s], xv[s], acc, 0, 0, 0);
  }
  if (!mok) return;
  float* crow = a.out + (int64_t)m * a.ldc;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int nb = n0 + 8 * g + 4 * hf;
    if (nb >= a.N) continue;
    f32x4 v = {acc[4 * g] * a.alpha, acc[4 * g + 1] * a.alpha, acc[4 * g + 2] * a.alpha, acc[4 * g + 3] * a.alpha};
    if (a.bias) v = v + *(const f32x4*)(a.bias + nb);
    if (a.add) v = v + *(const f32x4*)(a.add + (int64_t)m * a.ld_add + nb);
    if (a.act != ANIMA_ACT_NONE) {
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = apply_act(v[i], a.act);
    }
    f32x4* c = (f32x4*)(crow + nb);
    if (a.epi == ANIMA_EPI_STORE) {
      *c = v;
    } else if (a.epi == ANIMA_EPI_RESID) {
      *c = *c + v;
    } else {
      const f32x4 gt = *(const f32x4*)(a.gate + a.gate_off + nb);
      const f32x4 o = *c;
      f32x4 r;
#pragma unroll
      for (int i = 0; i < 4; i++) r[i] = __builtin_fmaf(gt[i], v[i], o[i]);
      *c = r;
    }
  }
}

// Tall-skinny fp32 product (the LoRA A side: N = stacked rank <= 128, K = model width): HBM-bound
// on x, so one x tile feeds RT column tiles of 32, and eight waves split the k-tiles (wave w takes
// k-tiles w, w + 8, ...) to keep enough loads in flight; the partial sums are added in a fixed
// tree order through LDS (deterministic).  Block: 32 rows x 32 RT columns.  Lane layout and
// epilogue as gemm_f32m_kernel.
constexpr int SK_WAVES = 8;
template <int RT, bool BF>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_f32m_skinny_kernel(F32WArgs a) {
  __shared__ float part[SK_WAVES / 2 * 64 * 16 * RT];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lq = lane & 31, hf = lane >> 5;
  const int m0 = blockIdx.y * 32, nb = blockIdx.x * 32 * RT;
  const int m = m0 + lq;
  const bool mok = m < a.M;
  const float* xr = a.x + (int64_t)(mok ? m : 0) * a.ldx + 16 * hf;
  int64_t wr[RT];
  bool nok[RT];
#pragma unroll
  for (int t = 0; t < RT; t++) {
    const int n = nb + 32 * t + lq;
    nok[t] = n < a.N;
    wr[t] = (int64_t)(nok[t] ? n : 0) * a.K + 16 * hf;
  }
  f32x16 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; t++) acc[t] = f32x16{};
  // k-tile loads; the loop issues tile i + 1's loads before tile i's MFMAs (register double buffer)
  auto load = [&](int kt, float4 (&xv)[4], float4 (&wv)[RT][4]) {
    const int k0 = 32 * kt;
    if (k0 + 32 <= a.K) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (RT <= 3) {  // unconditional in-bounds loads (rows clamped), then selects
          const float4 x0 = *(const float4*)(xr + k0 + 4 * j);
          xv[j] = mok ? x0 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
          for (int t = 0; t < RT; t++) {
            const float4 w0 = ld_w4<BF>(a.w, wr[t] + k0 + 4 * j);
            wv[t][j] = nok[t] ? w0 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          }
        } else {  // (the temporaries of the select form would not fit in registers)
          xv[j] = mok ? *(const float4*)(xr + k0 + 4 * j) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
          for (int t = 0; t < RT; t++)
            wv[t][j] = nok[t] ? ld_w4<BF>(a.w, wr[t] + k0 + 4 * j) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
      }
    } else {  // the last, partial k-tile
      float xs[16], ws[RT][16];
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const bool kok = k0 + 16 * hf + s < a.K;
        xs[s] = mok && kok ? xr[k0 + s] : 0.0f;
#pragma unroll
        for (int t = 0; t < RT; t++) ws[t][s] = nok[t] && kok ? ld_w1<BF>(a.w, wr[t] + k0 + s) : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        xv[j] = make_float4(xs[4 * j], xs[4 * j + 1], xs[4 * j + 2], xs[4 * j + 3]);
#pragma unroll
        for (int t = 0; t < RT; t++) wv[t][j] = make_float4(ws[t][4 * j], ws[t][4 * j + 1], ws[t][4 * j + 2], ws[t][4 * j + 3]);
      }
    }
  };
  auto mma = [&](const float4 (&xv)[4], const float4 (&wv)[RT][4]) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int t = 0; t < RT; t++) {
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[j].x, wv[t][j].x, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[j].y, wv[t][j].y, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[j].z, wv[t][j].z, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[j].w, wv[t][j].w, acc[t], 0, 0, 0);
      }
  };
  const int nkt = (a.K + 31) / 32;
  if (wave < nkt) {
    float4 xa[4], wa[RT][4], xb[4], wb[RT][4];
    load(wave, xa, wa);
    int kt = wave;
    for (;;) {
      const bool more = kt + SK_WAVES < nkt;
      if (more) load(kt + SK_WAVES, xb, wb);
      mma(xa, wa);
      if (!more) break;
      kt += SK_WAVES;
      const bool more2 = kt + SK_WAVES < nkt;
      if (more2) load(kt + SK_WAVES, xa, wa);
      mma(xb, wb);
      if (!more2) break;
      kt += SK_WAVES;
    }
  }
  // tree reduction: waves [h, 2h) hand their sums to waves [0, h), h = 4, 2, 1
#pragma unroll
  for (int h = SK_WAVES / 2; h >= 1; h >>= 1) {
    if (wave >= h && wave < 2 * h) {
#pragma unroll
      for (int t = 0; t < RT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) part[(((wave - h) * RT + t) * 64 + lane) * 16 + r] = acc[t][r];
    }
    __syncthreads();
    if (wave < h) {
#pragma unroll
      for (int t = 0; t < RT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = acc[t][r] + part[((wave * RT + t) * 64 + lane) * 16 + r];
    }
    __syncthreads();
  }
  if (wave > 0) return;
#pragma unroll
  for (int t = 0; t < RT; t++) {
    if (!nok[t]) continue;
    const int n = nb + 32 * t + lq;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int mm = m0 + 8 * (r >> 2) + 4 * hf + (r & 3);
      if (mm >= a.M) continue;
      float v = acc[t][r] * a.alpha;
      if (a.bias) v = v + a.bias[n];
      if (a.add) v = v + a.add[(int64_t)mm * a.ld_add + n];
      v = apply_act(v, a.act);
      float* c = a.out + (int64_t)mm * a.ldc + n;
      if (a.epi == ANIMA_EPI_STORE) *c = v;
      else if (a.epi == ANIMA_EPI_RESID) *c = *c + v;
      else *c = __builtin_fmaf(a.gate[a.gate_off + n], v, *c);
    }
  }
}

// ------------------------------------------------------------------ split-bf16 products
//
// ANIMA_W_F32S3: an fp32 matrix stored as three bf16 planes w0 + w1 + w2 (each the bf16 rounding of
// what the previous planes leave; the differences are exact in fp32, so |w - w0 - w1 - w2| <=
// 2^-24 |w|).  The activations are split the same way in registers, and x.w = sum_{i+j<=2} x_i w_j
// (the dropped terms are below 2^-24 of the product) runs as six v_mfma_f32_32x32x16_bf16 per
// 16-k slice with fp32 accumulation: fp32-level accuracy at about a third of the fp32 matrix-core
// time.  Both operands of one MFMA hold k = 8h .. 8h + 7 in lane half h, so the k order is the same
// on both sides.  Output layouts and epilogues are those of the fp32 kernels.


// acc += sum_{i+j<=2} a_i b_j on the 16x16x32 bf16 shape, smallest terms first
__device__ __forceinline__ f32x4 mfma16_s3(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], acc, 0, 0, 0);
}

constexpr int TK_WAVES = 8;
constexpr int TK_XB = 32 * 128;  // one wave's x step tile: 32 rows x 32 fp32 (int8 x: 32 rows x 32 bytes)

// Per-lane DMA state of gemm_s3_tall_kernel: x instruction i covers rows 8 i .. 8 i + 7 of the wave
// (lane -> row 8 i + lane / 8, piece slot lane % 8 holding k-piece (slot ^ row) % 8 of 4 fp32); W
// instruction t covers plane t / CT, rows 16 (t % CT) .. + 15 (lane -> row + lane / 4, slot
// lane % 4 holding k-piece slot ^ ((row / 2) % 4) of 8 bf16), issued by wave t % TK_WAVES.
// int8 x (Q8): one instruction for the wave's 32 rows x 32 bytes, lane -> row lane / 2, slot
// lane % 2 holding the row's 16-byte half (slot ^ q8_swz(row)).
template <int RT, bool Q8>
struct TallDma {
  static constexpr int CT = 2 * RT, WI = (6 * RT + TK_WAVES - 1) / TK_WAVES, XI = Q8 ? 1 : 4;
  static constexpr int XB = Q8 ? 1024 : TK_XB;  // one wave's x bytes per step
  __amdgpu_buffer_rsrc_t rx, rw;
  int xo[XI], xk[XI], wo[WI], wk[WI];
};

// the 16-byte halves of rows 8 .. 15 (mod 16) trade places, so that a half-wave's 8-byte reads
// (16 rows, two k-groups) touch every bank once
__device__ __forceinline__ int q8_swz(int row) { return (row >> 3) & 1; }

// One step's copies into `buf` (restrict: the compiler then tells them apart from the operand
// reads of the other buffer and does not make those reads wait for them).
template <int RT, bool Q8>
__device__ __forceinline__ void tall_issue(const TallDma<RT, Q8>& d, char* __restrict__ buf, int k0, int K, int wave) {
  using D = TallDma<RT, Q8>;
#pragma unroll
  for (int i = 0; i < D::XI; i++)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(d.rx, (lds_void_t*)(buf + wave * D::XB + i * 1024), 16,
                                             k0 + d.xk[i] < K ? d.xo[i] + (Q8 ? 1 : 4) * k0 : 0x7ffffff0, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < D::WI; j++) {
    const int t = wave + TK_WAVES * j;
    if (t < 6 * RT)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(d.rw, (lds_void_t*)(buf + TK_WAVES * D::XB + t * 1024), 16,
                                               k0 + d.wk[j] < K ? d.wo[j] + 2 * k0 : 0x7ffffff0, 0, 0, 0);
  }
}

// eight int8 values as bf16 (exact: at most 8 significant bits)
__device__ __forceinline__ bf16x8 i8x8_bf16(uint32_t lo, uint32_t hi) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    o[e] = (bf16)(float)(int8_t)(lo >> (8 * e));
    o[4 + e] = (bf16)(float)(int8_t)(hi >> (8 * e));
  }
  return o;
}

// acc += sum_j a b_j on the 16x16x32 shape (a exact in bf16), smallest terms first
__device__ __forceinline__ f32x4 mfma16_q3(const bf16x8& a, const bf16x8 (&b)[3], f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[1], acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[0], acc, 0, 0, 0);
}

// One step's operand reads from `buf` and its products (lane (r16, g): x row 16 i + r16, W row
// 16 t + r16, k = 8 g .. 8 g + 7 of the step on both operands).
template <int RT, bool Q8>
__device__ __forceinline__ void tall_step(const char* __restrict__ buf, int wave, int r16, int g, f32x4 (&acc)[2][2 * RT]) {
  using D = TallDma<RT, Q8>;
  constexpr int CT = 2 * RT;
  bf16x8 wv[CT][3];
#pragma unroll
  for (int t = 0; t < CT; t++) {
    const int row = 16 * t + r16;
#pragma unroll
    for (int p = 0; p < 3; p++)
      wv[t][p] = *(const bf16x8*)(buf + TK_WAVES * D::XB + p * CT * 1024 + row * 64 + 16 * (g ^ ((row >> 1) & 3)));
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int row = 16 * i + r16;
    if constexpr (Q8) {
      const char* xr = buf + wave * D::XB + 16 * (2 * row + ((g >> 1) ^ q8_swz(row))) + 8 * (g & 1);
      typedef int i32x2 __attribute__((ext_vector_type(2)));
      i32x2 v = *(const i32x2*)xr;
      asm volatile("" : "+v"(v));
      const bf16x8 xb = i8x8_bf16((uint32_t)v[0], (uint32_t)v[1]);
#pragma unroll
      for (int t = 0; t < CT; t++) acc[i][t] = mfma16_q3(xb, wv[t], acc[i][t]);
    } else {
      const char* xr = buf + wave * D::XB + row * 128;
      // whole 16-byte reads: split into scalar loads and merged again, the reads lose the alias
      // information that keeps them from waiting on the other buffer's copies
      f32x4 v0 = *(const f32x4*)(xr + 16 * ((2 * g) ^ (row & 7)));
      f32x4 v1 = *(const f32x4*)(xr + 16 * ((2 * g + 1) ^ (row & 7)));
      asm volatile("" : "+v"(v0), "+v"(v1));
      const float4 x0 = make_float4(v0[0], v0[1], v0[2], v0[3]), x1 = make_float4(v1[0], v1[1], v1[2], v1[3]);
      bf16x8 xs[3];
      split3(x0, x1, xs);
#pragma unroll
      for (int t = 0; t < CT; t++) acc[i][t] = mfma16_s3(xs, wv[t], acc[i][t]);
    }
  }
}

// k-sliced tall-skinny split product (the stacked LoRA A side over many rows): a workgroup is 8
// waves x 32 rows (256 rows) over one slice of k, 32 k per step.  Both operands move HBM/L2 ->
// LDS with `buffer_load ... lds`, lane-contiguous 16-byte pieces (whole cache lines per
// instruction): x as each wave's 32 rows x 128 bytes, W as the step's 32 RT rows x 64 bytes of
// each plane, loaded once per workgroup and read by all eight waves.  (Register loads straight
// into the 16x16x32 operand layout touch 16-32 rows per instruction, one 16-byte access each,
// which bounds that form by the vector memory address path at half the HBM rate.)  Pieces are
// XOR-swizzled within their row so that the operand reads (8 lanes = 8 rows per 16-byte access)
// hit distinct bank groups.  Up to four step buffers, one barrier per step.  Each slice writes its
// partial sums [slice][M][N]; s3_ksum_kernel adds them in slice order (deterministic) and applies
// the epilogue.  Offsets past a buffer's end read zeros: the k tail and rows past M.  A row of W
// past N reads other rows' data (or zeros) and feeds only columns that are never stored.
// Q8: x is per-token int8 (a.xq, row stride a.ldx bytes, K % 16 == 0), each wave's 32 rows x 32
// bytes one copy per step, the bytes widened to bf16 (exact) for three MFMAs per tile against the
// three planes; the sum pass applies the row scales a.xs.
template <int RT, bool Q8>
__global__ __launch_bounds__(64 * TK_WAVES) void gemm_s3_tall_kernel(F32WArgs a, float* part, int spb) {
  using D = TallDma<RT, Q8>;
  constexpr int CT = 2 * RT;
  constexpr int BUF = TK_WAVES * D::XB + 3 * CT * 1024;
  // step buffers: as many as fit in LDS (up to 4), so that up to TD - 1 steps' copies are in
  // flight behind the one being computed
  constexpr int TD = 160 * 1024 / BUF < 4 ? 160 * 1024 / BUF : 4;
  __shared__ __attribute__((aligned(1024))) char smem[TD * BUF];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int nb = blockIdx.x * 32 * RT, m0 = blockIdx.y * (32 * TK_WAVES) + wave * 32;
  const int nst = (a.K + 31) / 32, s0 = blockIdx.z * spb, s1 = nst < s0 + spb ? nst : s0 + spb;
  // (wave-uniform values taken to scalar registers: a buffer resource in vector registers would
  // turn every load into a loop over the lanes' distinct values)
  const int rows = __builtin_amdgcn_readfirstlane(a.M - m0 < 0 ? 0 : a.M - m0 < 32 ? a.M - m0 : 32);
  const int mb = __builtin_amdgcn_readfirstlane(rows ? m0 : 0);
  D d;
  d.rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)(2 * (2 * a.wplane + (int64_t)a.N * a.K)), 0x00020000);
  if constexpr (Q8) {
    d.rx = __builtin_amdgcn_make_buffer_rsrc((void*)(a.xq + (int64_t)mb * a.ldx), (short)0, rows * (int)a.ldx, 0x00020000);
    const int row = lane >> 1, h = (lane & 1) ^ q8_swz(row);
    d.xk[0] = 16 * h;
    d.xo[0] = row * (int)a.ldx + 16 * h;
  } else {
    d.rx = __builtin_amdgcn_make_buffer_rsrc((void*)(a.x + (int64_t)mb * a.ldx), (short)0, rows * (int)a.ldx * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = 8 * i + (lane >> 3), c = (lane & 7) ^ (row & 7);
      d.xk[i] = 4 * c;
      d.xo[i] = (row * (int)a.ldx + 4 * c) * 4;
    }
  }
#pragma unroll
  for (int j = 0; j < D::WI; j++) {
    const int t = wave + TK_WAVES * j, tt = t < 6 * RT ? t : 0;
    const int p = tt / CT, row = 16 * (tt % CT) + (lane >> 2), c = (lane & 3) ^ ((row >> 1) & 3);
    d.wk[j] = 8 * c;
    const int64_t o = p * 2 * a.wplane + ((int64_t)(nb + row) * a.K + 8 * c) * 2;
    d.wo[j] = o < 0x7ffffff0 ? (int)o : 0x7ffffff0;  // (past the end: reads zeros)
  }
  f32x4 acc[2][CT];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int t = 0; t < CT; t++) acc[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // Copies issued by this wave per step: 4 of x (1 of int8 x) and its share of the 6 RT of W (waves below
  // (6 RT) % 8, or all when it is 0, take one more).  Steps s0 .. s0 + TD - 2 are issued up front
  // and step st + TD - 1 after the barrier of step st, so before step st the TD - 2 steps after it
  // are in flight (once they exist) and may stay so: vmcnt((TD - 2) * per-step count), vmcnt(0)
  // in the last steps of the slice.
  constexpr int WHI = (6 * RT) % TK_WAVES ? (6 * RT) % TK_WAVES : TK_WAVES;
  constexpr int CHI = D::XI + D::WI, NHI = (TD - 2) * CHI, NLO = (TD - 2) * (CHI - 1);
  static_assert(TD >= 2, "two step buffers at least");
  static_assert(NHI < 64, "vmcnt field");
  for (int i = 0; i < TD - 1; i++)
    if (s0 + i < s1) tall_issue<RT, Q8>(d, smem + i * BUF, 32 * (s0 + i), a.K, wave);
  for (int st = s0; st < s1; st++) {
    if (st + TD - 1 <= s1) {  // steps st + 1 .. st + TD - 2 all exist (and are issued)
      if (wave < WHI) __builtin_amdgcn_s_waitcnt((NHI & 15) | (7 << 4) | (15 << 8) | ((NHI >> 4) << 14));
      else __builtin_amdgcn_s_waitcnt((NLO & 15) | (7 << 4) | (15 << 8) | ((NLO >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt((15 << 8) | (7 << 4));  // vmcnt(0)
    }
    // every wave's copies of step st have landed, and every wave is done reading step st - 1's
    // buffer, which step st + TD - 1 then refills
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int nx = st + TD - 1;
    if (nx < s1) tall_issue<RT, Q8>(d, smem + ((nx - s0) % TD) * BUF, 32 * nx, a.K, wave);
    tall_step<RT, Q8>(smem + ((st - s0) % TD) * BUF, wave, r16, g, acc);
  }
  // lane (r16, g) holds rows 16 i + 4 g + r of column tile t's column r16
  float* pp = part + (int64_t)blockIdx.z * a.M * a.N;
#pragma unroll
  for (int t = 0; t < CT; t++) {
    const int n = nb + 16 * t + r16;
    if (n >= a.N) continue;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + 16 * i + 4 * g + r;
        if (m < a.M) pp[(int64_t)m * a.N + n] = acc[i][t][r];
      }
  }
}

// The slices' partial sums added in slice order, then the row scale (int8 x), alpha, bias, add,
// activation and the store / residual / gated epilogue of the split-weight kernels; four
// consecutive (flat [M][N]) outputs per thread with 16-byte partial reads, every slice's read
// issued before the sums (element by element when M * N % 4 != 0).
__global__ __launch_bounds__(256) void s3_ksum_kernel(F32WArgs a, const float* part, int ks) {
  const int64_t i4 = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x), mn = (int64_t)a.M * a.N;
  if (i4 >= mn) return;
  constexpr int KSM = 16;
  f32x4 v;
  if (mn % 4 == 0) {  // (every slice's plane then starts 16-byte aligned)
    f32x4 pv[KSM];
#pragma unroll
    for (int s = 0; s < KSM; s++)
      if (s < ks) pv[s] = *(const f32x4*)(part + s * mn + i4);
    v = pv[0];
#pragma unroll
    for (int s = 1; s < KSM; s++)
      if (s < ks) v = v + pv[s];
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float t = 0.0f;
      if (i4 + e < mn) {
        t = part[i4 + e];
        for (int s = 1; s < ks; s++) t = t + part[s * mn + i4 + e];
      }
      v[e] = t;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int64_t idx = i4 + e;
    if (idx >= mn) break;
    const int m = (int)(idx / a.N), n = (int)(idx - (int64_t)m * a.N);
    float r = (a.xs ? v[e] * a.xs[m] : v[e]) * a.alpha;
    if (a.bias) r = r + a.bias[n];
    if (a.add) r = r + a.add[(int64_t)m * a.ld_add + n];
    r = apply_act(r, a.act);
    float* c = a.out + (int64_t)m * a.ldc + n;
    if (a.epi == ANIMA_EPI_STORE) *c = r;
    else if (a.epi == ANIMA_EPI_RESID) *c = *c + r;
    else *c = __builtin_fmaf(a.gate[a.gate_off + n], r, *c);
  }
}

// Split product with the operands swapped (the LoRA B side, K = rank): the C^T layout and 16-byte
// epilogue of gemm_f32m_t_kernel.  A wave owns 32 rows x 32 NT columns (NT MFMA tiles sharing one
// split of x, so a wave reads each x row once for NT tiles); workgroup = 2 x 2 waves.
template <int NT>
__global__ __launch_bounds__(256) void gemm_s3_t_kernel(F32WArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lq = lane & 31, hf = lane >> 5;
  const int m0 = blockIdx.y * 64 + (wave & 1) * 32;
  const int n0 = blockIdx.x * 64 * NT + (wave >> 1) * 32 * NT;
  const int m = m0 + lq;
  const bool mok = m < a.M;
  const float* xr = a.x + (int64_t)(mok ? m : 0) * a.ldx + 8 * hf;
  const uint16_t* W = (const uint16_t*)a.w;
  const int64_t plane = a.wplane;
  int64_t wr[NT];
  bool nok[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int n = n0 + 32 * t + lq;
    nok[t] = n < a.N;
    wr[t] = (int64_t)(nok[t] ? n : 0) * a.K + 8 * hf;
  }
  const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  f32x16 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = f32x16{};
  for (int k0 = 0; k0 < a.K; k0 += 32) {  // two 16-k slices per load round trip
    float4 x[2][2];
    bf16x8 wv[NT][2][3], xs[3];
    // unconditional loads at clamped in-bounds offsets, taken as loaded: rows past M or N only
    // reach outputs that are not stored; a lane whose 8 values of a slice lie past K (K % 8 == 0:
    // all in or all out) loads its row's first 8 (xr and wr already hold the lane's 8 hf, so the
    // offset is -8 hf) and its x values are zeroed where they are split
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int k = k0 + 16 * h;
      const int kc = k + 8 * hf < a.K ? k : -8 * hf;
      x[h][0] = *(const float4*)(xr + kc);
      x[h][1] = *(const float4*)(xr + kc + 4);
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int p = 0; p < 3; p++) wv[t][h][p] = ld_bf8(W + p * plane + wr[t] + kc);
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const bool kok = k0 + 16 * h + 8 * hf < a.K;
      split3(kok ? x[h][0] : z4, kok ? x[h][1] : z4, xs);
#pragma unroll
      for (int t = 0; t < NT; t++) acc[t] = mfma_s3(wv[t][h], xs, acc[t]);
    }
  }
  if (!mok) return;
  float* crow = a.out + (int64_t)m * a.ldc;
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int nbk = n0 + 32 * t + 8 * g + 4 * hf;
      if (nbk >= a.N) continue;
      f32x4 v = {acc[t][4 * g] * a.alpha, acc[t][4 * g + 1] * a.alpha, acc[t][4 * g + 2] * a.alpha,
                 acc[t][4 * g + 3] * a.alpha};
      if (a.bias) v = v + *(const f32x4*)(a.bias + nbk);
      if (a.add) v = v + *(const f32x4*)(a.add + (int64_t)m * a.ld_add + nbk);
      if (a.act != ANIMA_ACT_NONE) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = apply_act(v[i], a.act);
      }
      f32x4* c = (f32x4*)(crow + nbk);
      if (a.epi == ANIMA_EPI_STORE) {
        *c = v;
      } else if (a.epi == ANIMA_EPI_RESID) {
        *c = *c + v;
      } else {
        const f32x4 gt = *(const f32x4*)(a.gate + a.gate_off + nbk);
        const f32x4 o = *c;
        f32x4 r;
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = __builtin_fmaf(gt[i], v[i], o[i]);
        *c = r;
      }
    }
  }
}

// fp32 activations x bf16 weights on the bf16 matrix cores (the text encoder's and the LLM
// adapter's linears, app/gpu/gemm.js:17-55 semantics: fp32 products and sums of the bf16 weights).
// x enters as its three bf16 terms (x = h + m + l exactly), the weight as it is, so every product
// term is exact in fp32 and the MFMA sums are fp32: three bf16 MFMAs per 32x32x16 step in place of
// eight fp32 ones (v_mfma_f32_32x32x2_f32).  W rows are the MFMA A operand (the C^T layout and
// 16-byte epilogue of gemm_f32m_t_kernel).  A wave owns 32 rows x 64 columns (two MFMA tiles that
// share one split of x); a workgroup is 2 column waves x KG k-groups over a 32 x 128 tile, k-group g
// takes the 32-k chunks g, g + KG, ... (the next chunk's loads issued before this chunk's MFMAs),
// and the k-groups' partial sums are added in a fixed tree order through LDS (deterministic).
// Needs K % 32 == 0, N % 4 == 0 and 16-byte aligned x / W / out / bias / add / gate rows.
template <int KG>
__global__ __launch_bounds__(128 * KG) void gemm_bf16_s3_kernel(F32WArgs a) {
  __shared__ float part[(KG > 1 ? KG / 2 : 1) * 2 * 32 * 64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lq = lane & 31, hf = lane >> 5;
  const int wn = wave & 1, kg = wave >> 1;
  const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 128 + wn * 64;
  const int m = m0 + lq;
  const bool mok = m < a.M;
  const float* xr = a.x + (int64_t)(mok ? m : 0) * a.ldx + 8 * hf;
  const uint16_t* W = (const uint16_t*)a.w;
  int64_t wr[2];
  bool nok[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int n = n0 + 32 * t + lq;
    nok[t] = n < a.N;
    wr[t] = (int64_t)(nok[t] ? n : 0) * a.K + 8 * hf;
  }
  f32x16 acc[2] = {f32x16{}, f32x16{}};
  const int nch = a.K / 32;
  // chunk J: lane (l, h) loads x[m][32J + 16s + 8h .. +7] and W[n_t][same] for s = 0, 1.  Rows
  // past M or N are clamped to row 0 and used as they are: such an x row only reaches output row
  // m, such a W row only output column n, and neither is stored.
#define B3_LOAD(J, X, WV)                                                        \
  {                                                                              \
    const int k_ = 32 * (J);                                                     \
    _Pragma("unroll") for (int s = 0; s < 2; s++) {                              \
      X[2 * s] = *(const float4*)(xr + k_ + 16 * s);                             \
      X[2 * s + 1] = *(const float4*)(xr + k_ + 16 * s + 4);                     \
      _Pragma("unroll") for (int t = 0; t < 2; t++) WV[t][s] = ld_bf8(W + wr[t] + k_ + 16 * s); \
    }                                                                            \
  }
  // smallest terms first: l, m, h
#define B3_MMA(X, WV)                                                                          \
  {                                                                                            \
    _Pragma("unroll") for (int s = 0; s < 2; s++) {                                            \
      bf16x8 xs_[3];                                                                           \
      split3(X[2 * s], X[2 * s + 1], xs_);                                                     \
      _Pragma("unroll") for (int p = 2; p >= 0; p--)                                           \
      _Pragma("unroll") for (int t = 0; t < 2; t++)                                            \
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(WV[t][s], xs_[p], acc[t], 0, 0, 0);   \
    }                                                                                          \
  }
  int j = kg;
  if (j < nch) {
    float4 xa[4], xb[4];
    bf16x8 wa[2][2], wb[2][2];
    B3_LOAD(j, xa, wa)
    for (;;) {
      B3_LOAD(min(j + KG, nch - 1), xb, wb)
      B3_MMA(xa, wa)
      j += KG;
      if (j >= nch) break;
      B3_LOAD(min(j + KG, nch - 1), xa, wa)
      B3_MMA(xb, wb)
      j += KG;
      if (j >= nch) break;
    }
  }
#undef B3_LOAD
#undef B3_MMA
  if constexpr (KG > 1) {
    // k-groups [h, 2h) hand their sums to k-groups [0, h); consecutive lanes on consecutive words
#pragma unroll
    for (int h = KG / 2; h >= 1; h >>= 1) {
      if (kg >= h && kg < 2 * h) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int r = 0; r < 16; r++) part[((((kg - h) * 2 + wn) * 2 + t) * 16 + r) * 64 + lane] = acc[t][r];
      }
      __syncthreads();
      if (kg < h) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int r = 0; r < 16; r++) acc[t][r] = acc[t][r] + part[(((kg * 2 + wn) * 2 + t) * 16 + r) * 64 + lane];
      }
      __syncthreads();
    }
  }
  if (kg > 0 || !mok) return;
  float* crow = a.out + (int64_t)m * a.ldc;
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int nb = n0 + 32 * t + 8 * g + 4 * hf;
      if (nb >= a.N) continue;
      f32x4 v = {acc[t][4 * g] * a.alpha, acc[t][4 * g + 1] * a.alpha, acc[t][4 * g + 2] * a.alpha,
                 acc[t][4 * g + 3] * a.alpha};
      if (a.bias) v = v + *(const f32x4*)(a.bias + nb);
      if (a.add) v = v + *(const f32x4*)(a.add + (int64_t)m * a.ld_add + nb);
      if (a.act != ANIMA_ACT_NONE) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = apply_act(v[i], a.act);
      }
      f32x4* c = (f32x4*)(crow + nb);
      if (a.epi == ANIMA_EPI_STORE) {
        *c = v;
      } else if (a.epi == ANIMA_EPI_RESID) {
        *c = *c + v;
      } else {
        const f32x4 gt = *(const f32x4*)(a.gate + a.gate_off + nb);
        const f32x4 o = *c;
        f32x4 r;
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = __builtin_fmaf(gt[i], v[i], o[i]);
        *c = r;
      }
    }
}

// The same product (x in three bf16 terms x bf16 weights) for grids of at least 128 workgroups: a
// workgroup (2 x 2 waves, each 32 rows x 64 columns) computes a 64 x 128 tile with both operand
// tiles staged through double-buffered LDS, 32 k per step (x split once per workgroup as it is
// stored; each x row read from memory once per 128 columns and each weight row once per 64 rows,
// where the register-operand kernel reads them once per wave).  LDS rows of 40 bf16 (80 bytes)
// give conflict-free 16-byte fragment reads.  Epilogue and C^T layout of gemm_bf16_s3_kernel.
constexpr int B3L_ROW = 40;
__global__ __launch_bounds__(256) void gemm_bf16_s3_lds_kernel(F32WArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 xs[2][3][64 * B3L_ROW];
  __shared__ __attribute__((aligned(16))) bf16 wsm[2][128 * B3L_ROW];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63, lq = lane & 31, hf = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int mb = blockIdx.y * 64, nb = blockIdx.x * 128;
  // loader roles: x row t/4, k (t%4)*8 .. +7; weight row t/2, k (t%2)*16 .. +15 (rows past M / N
  // clamped to row 0: they only reach outputs that are not stored)
  const int xr_row = t >> 2, xk = (t & 3) * 8, wr_row = t >> 1, wk = (t & 1) * 16;
  // blockIdx.z: k-slice z of a split product (x + z x_gs, w + z w_gs, partial output out + z out_gs)
  const int z = blockIdx.z;
  const int64_t ldw = a.ldw ? a.ldw : a.K;
  const float* xsrc = a.x + z * a.x_gs + (int64_t)(mb + xr_row < a.M ? mb + xr_row : 0) * a.ldx + xk;
  const uint16_t* wsrc = (const uint16_t*)a.w + z * a.w_gs + (int64_t)(nb + wr_row < a.N ? nb + wr_row : 0) * ldw + wk;
  float4 xv0, xv1;
  uint4 wv0, wv1;
  auto load = [&](int k0) {
    xv0 = *(const float4*)(xsrc + k0);
    xv1 = *(const float4*)(xsrc + k0 + 4);
    wv0 = *(const uint4*)(wsrc + k0);
    wv1 = *(const uint4*)(wsrc + k0 + 8);
  };
  auto store = [&](int st) {
    bf16x8 sp[3];
    split3(xv0, xv1, sp);
#pragma unroll
    for (int p = 0; p < 3; p++) *(bf16x8*)(&xs[st][p][xr_row * B3L_ROW + xk]) = sp[p];
    *(uint4*)(&wsm[st][wr_row * B3L_ROW + wk]) = wv0;
    *(uint4*)(&wsm[st][wr_row * B3L_ROW + wk + 8]) = wv1;
  };
  f32x16 acc[2] = {f32x16{}, f32x16{}};
  const int nch = a.K / 32;
  load(0);
  store(0);
  __syncthreads();
  for (int kc = 0; kc < nch; kc++) {
    const int st = kc & 1;
    if (kc + 1 < nch) load(32 * (kc + 1));
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int ko = 16 * s + 8 * hf;
      bf16x8 fw[2], fx[3];
#pragma unroll
      for (int u = 0; u < 2; u++) fw[u] = *(const bf16x8*)(&wsm[st][(wn * 64 + 32 * u + lq) * B3L_ROW + ko]);
#pragma unroll
      for (int p = 0; p < 3; p++) fx[p] = *(const bf16x8*)(&xs[st][p][(wm * 32 + lq) * B3L_ROW + ko]);
      // smallest terms first: l, m, h
#pragma unroll
      for (int p = 2; p >= 0; p--)
#pragma unroll
        for (int u = 0; u < 2; u++) acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fw[u], fx[p], acc[u], 0, 0, 0);
    }
    if (kc + 1 < nch) store(st ^ 1);
    __syncthreads();
  }
  const int m = mb + wm * 32 + lq;
  if (m >= a.M) return;
  float* crow = a.out + z * a.out_gs + (int64_t)m * a.ldc;
  const int n0 = nb + wn * 64;
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int nbk = n0 + 32 * u + 8 * g + 4 * hf;
      if (nbk >= a.N) continue;
      f32x4 v = {acc[u][4 * g] * a.alpha, acc[u][4 * g + 1] * a.alpha, acc[u][4 * g + 2] * a.alpha,
                 acc[u][4 * g + 3] * a.alpha};
      if (a.bias) v = v + *(const f32x4*)(a.bias + nbk);
      if (a.add) v = v + *(const f32x4*)(a.add + (int64_t)m * a.ld_add + nbk);
      if (a.act != ANIMA_ACT_NONE) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = apply_act(v[i], a.act);
      }
      f32x4* c = (f32x4*)(crow + nbk);
      if (a.epi == ANIMA_EPI_STORE) {
        *c = v;
      } else if (a.epi == ANIMA_EPI_RESID) {
        *c = *c + v;
      } else {
        const f32x4 gt = *(const f32x4*)(a.gate + a.gate_off + nbk);
        const f32x4 o = *c;
        f32x4 r;
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = __builtin_fmaf(gt[i], v[i], o[i]);
        *c = r;
      }
    }
}

// The epilogue of a split-k product: out = epilogue(alpha * sum_z P[z] + bias + add) with the act
// and store / residual / gated forms of the linear epilogues, one element per thread.
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const float* P, int ks, F32WArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, n_el = (int64_t)a.M * a.N;
  if (i >= n_el) return;
  const int64_t m = i / a.N;
  const int n = (int)(i - m * a.N);
  float acc = P[i];
  for (int z = 1; z < ks; z++) acc = acc + P[z * n_el + i];
  float v = acc * a.alpha;
  if (a.bias) v = v + a.bias[n];
  if (a.add) v = v + a.add[m * a.ld_add + n];
  v = apply_act(v, a.act);
  float* c = a.out + m * a.ldc + n;
  if (a.epi == ANIMA_EPI_STORE) *c = v;
  else if (a.epi == ANIMA_EPI_RESID) *c = *c + v;
  else *c = __builtin_fmaf(a.gate[a.gate_off + n], v, *c);
}

// Per-token int8 rows back to fp32, x[m][k] = q[m][k] * s[m] (one 4-byte group per thread;
// K % 4 == 0, ldq % 4 == 0).
__global__ __launch_bounds__(256) void dequant_rows_kernel(const int8_t* q, int64_t ldq, const float* s, float* x, int64_t M,
                                                           int K) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, kq = K / 4;
  if (i >= M * kq) return;
  const int64_t m = i / kq;
  const int k = (int)(i - m * kq) * 4;
  const char4 v = *(const char4*)(q + m * ldq + k);
  const float sc = s[m];
  *(float4*)(x + m * K + k) = make_float4((float)v.x * sc, (float)v.y * sc, (float)v.z * sc, (float)v.w * sc);
}

__global__ __launch_bounds__(256) void split3_kernel(const float* src, uint16_t* dst, int64_t n8, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    bf16x8 o[3];
    split3(*(const float4*)(src + 8 * i), *(const float4*)(src + 8 * i + 4), o);
#pragma unroll
    for (int p = 0; p < 3; p++) __builtin_memcpy(dst + p * n + 8 * i, &o[p], 16);
  }
}

// Small-M (M <= 8) bf16-weight GEMV: one wave per output column n, lanes stride K in 8-element
// chunks, fp32 FMA, wave reduction (timestep / adaLN projections, M = 1).
constexpr int GEMV_MAXM = 8;
__global__ __launch_bounds__(256) void gemv_f32w_kernel(F32WArgs a) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= a.N) return;
  const int64_t grp = blockIdx.y;
  a.x += grp * a.x_gs;
  a.w = (const uint16_t*)a.w + grp * a.w_gs;
  if (a.bias) a.bias += grp * a.bias_gs;
  a.out += grp * a.out_gs;
  float acc[GEMV_MAXM];
#pragma unroll
  for (int m = 0; m < GEMV_MAXM; m++) acc[m] = 0.0f;
  const uint16_t* wr = (const uint16_t*)a.w + (int64_t)n * a.K;
  for (int k = lane * 8; k < a.K; k += 512) {
    const uint4 wv = *(const uint4*)(wr + k);
    float wf[8];
    const uint32_t u[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      wf[2 * j] = __uint_as_float(u[j] << 16);
      wf[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
    }
#pragma unroll
    for (int m = 0; m < GEMV_MAXM; m++) {
      if (m >= a.M) break;
      const float4 x0 = *(const float4*)(a.x + (int64_t)m * a.ldx + k);
      const float4 x1 = *(const float4*)(a.x + (int64_t)m * a.ldx + k + 4);
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int j = 0; j < 8; j++) acc[m] = __builtin_fmaf(xv[j], wf[j], acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < GEMV_MAXM; m++) {
    if (m >= a.M) break;
    const float tot = wave_sum(acc[m]);
    if (lane == 0) {
      float r = tot * a.alpha;
      if (a.bias) r = r + a.bias[n];
      if (a.add) r = r + a.add[(int64_t)m * a.ld_add + n];
      r = apply_act(r, a.act);
      float* c = a.out + (int64_t)m * a.ldc + n;
      if (a.epi == ANIMA_EPI_STORE) *c = r;
      else if (a.epi == ANIMA_EPI_RESID) *c = *c + r;
      else *c = __builtin_fmaf(a.gate[a.gate_off + n], r, *c);
    }
  }
}

// ------------------------------------------------------------------ host

static bool al(const void* p, int b) { return ((uintptr_t)p & (b - 1)) == 0; }

int linear_launch(anima_ctx* c, const anima_linear_desc* d, int64_t s3_plane) {
  const anima_weight* W = d->W;
  if (!W) return fail(c, ANIMA_E_ARG, "anima_linear: null weight");
  const int64_t M = d->M;
  const int N = W->N, K = W->K;
  if (M < 0 || M > 0x7fffffff || N < 1 || K < 1) return fail(c, ANIMA_E_ARG, "anima_linear: M=%lld N=%d K=%d", (long long)M, N, K);
  if (!d->out || !W->w) return fail(c, ANIMA_E_ARG, "anima_linear: null out or weight data");
  if (d->act < ANIMA_ACT_NONE || d->act > ANIMA_ACT_SILU) return fail(c, ANIMA_E_ARG, "anima_linear: unknown act %d", d->act);
  if (d->epilogue < ANIMA_EPI_STORE || d->epilogue > ANIMA_EPI_GATED) return fail(c, ANIMA_E_ARG, "anima_linear: unknown epilogue %d", d->epilogue);
  if (d->epilogue == ANIMA_EPI_GATED && !d->gate) return fail(c, ANIMA_E_ARG, "anima_linear: gated epilogue without gate");
  const int64_t ldc = d->ldc ? d->ldc : N;
  if (ldc < N) return fail(c, ANIMA_E_ARG, "anima_linear: ldc=%lld < N=%d", (long long)ldc, N);
  const float alpha = d->alpha != 0.0f ? d->alpha : 1.0f;
  const int64_t ld_add = d->ld_add ? d->ld_add : N;
  if (d->add && ld_add < N) return fail(c, ANIMA_E_ARG, "anima_linear: ld_add=%lld < N=%d", (long long)ld_add, N);
  const bool lora = d->lora_xa || d->lora_b || d->lora_r;
  if (lora) {
    if (W->kind != ANIMA_W_I8 && W->kind != ANIMA_W_W4)
      return fail(c, ANIMA_E_UNSUPPORTED, "anima_linear: the LoRA epilogue takes i8 / w4 weights (kind %d)", W->kind);
    if (!d->lora_xa || !d->lora_b || d->lora_r < 16 || d->lora_r % 16 || d->ld_lora_xa < d->lora_r || d->ld_lora_xa % 4 ||
        !al(d->lora_xa, 16) || !al(d->lora_b, 16))
      return fail(c, ANIMA_E_ARG, "anima_linear: LoRA factors need lora_r %% 16 == 0 (%d), ld_lora_xa >= lora_r and %% 4 == 0 (%lld), 16-byte aligned",
                  d->lora_r, (long long)d->ld_lora_xa);
    if (d->lora_cols < 0 || (d->lora_cols && (N % d->lora_cols || d->lora_cols % 16)) ||
        d->ld_lora_xa < (int64_t)d->lora_r * (d->lora_cols ? N / d->lora_cols : 1))
      return fail(c, ANIMA_E_ARG, "anima_linear: lora_cols=%d must divide N=%d, be a multiple of 16 and fit ld_lora_xa=%lld",
                  d->lora_cols, N, (long long)d->ld_lora_xa);
    if (d->add) return fail(c, ANIMA_E_UNSUPPORTED, "anima_linear: the LoRA epilogue and an add term together");
  }
  if (M == 0) return ANIMA_OK;

  if (W->kind == ANIMA_W_F32S3) {
    // x: fp32 rows, or per-token int8 rows xq with their scales xs (y = xs[m] * (q W^T)[m])
    const bool q8 = d->xq != nullptr;
    if (q8 ? (d->x || !d->xs) : !d->x)
      return fail(c, ANIMA_E_ARG, "anima_linear: split weights need fp32 x, or int8 xq with its row scales xs (not both)");
    if (d->acc_out) return fail(c, ANIMA_E_ARG, "anima_linear: acc_out applies to i8/w4 weights only");
    const int64_t ldx = d->ldx ? d->ldx : K;
    if (ldx < K) return fail(c, ANIMA_E_ARG, "anima_linear: ldx < K");
    if (q8 ? (K % 16 || ldx % 16 || !al(d->xq, 16) || !al(W->w, 16)) : (K % 8 || ldx % 4 || !al(d->x, 16) || !al(W->w, 16)))
      return fail(c, ANIMA_E_ARG, "anima_linear: split weights need K %% 8 == 0, ldx %% 4 == 0, 16-byte aligned x and w "
                                  "(int8 x: K %% 16 == 0, ldx %% 16 == 0)");
    if (s3_plane && s3_plane < (int64_t)N * K) return fail(c, ANIMA_E_ARG, "anima_linear: split-weight plane stride below N * K");
    F32WArgs f{d->x, ldx, W->w, W->bias, d->out, ldc, alpha, d->act, d->epilogue, d->gate, d->gate_off,
               (int)M, N, K, 0, 0, 0, 0, d->add, ld_add, 0};
    f.wplane = s3_plane ? s3_plane : (int64_t)N * K;
    f.xq = d->xq;
    f.xs = d->xs;
    // the tall kernel's buffer offsets are 32-bit: 32 rows of x and the three planes of W;
    // N in (96, 256] runs as 64-column workgroups
    const bool skf = K >= 512 && ldx < (1 << 23) && 2 * (2 * f.wplane + (int64_t)N * K) < (1LL << 31) - 64 && N <= 256;
    if (q8 && !skf) {
      // int8 rows for a shape the tall kernel does not take: back to fp32 rows (pooled scratch,
      // x = q * s rounded once), then the fp32 path
      void* xf = nullptr;
      if (int rc = anima_alloc(c, (size_t)M * K * 4, &xf)) return rc;
      const int64_t groups = M * (K / 4);
      hipLaunchKernelGGL(dequant_rows_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, c->stream, d->xq, ldx,
                         d->xs, (float*)xf, M, K);
      anima_linear_desc dd = *d;
      dd.x = (const float*)xf;
      dd.ldx = K;
      dd.xq = nullptr;
      dd.xs = nullptr;
      const int rc = linear_launch(c, &dd, s3_plane);
      anima_free(c, xf);
      return rc;
    }
    Launch L(c, "gemm.f32s3", 2.0 * M * N * K, 0.0);
    if (skf) {
      // k-slices so that the grid gives every CU about one workgroup, each slice at least 4 steps
      const int srt = N <= 32 ? 1 : N <= 64 || N > 96 ? 2 : 3;
      const int cb = (N + 32 * srt - 1) / (32 * srt), rb = (int)((M + 32 * TK_WAVES - 1) / (32 * TK_WAVES));
      const int nst = (K + 31) / 32;
      int ks = (c->num_cus + cb * rb - 1) / (cb * rb);
      ks = ks < nst / 4 ? ks : nst / 4;
      ks = ks < 1 ? 1 : ks > 16 ? 16 : ks;  // (the sum pass holds up to 16 slices)
      const int spb = (nst + ks - 1) / ks;
      ks = (nst + spb - 1) / spb;
      void* pt = nullptr;
      if (int rc = anima_alloc(c, (size_t)ks * M * N * 4, &pt)) return rc;
      const dim3 tg((unsigned)cb, (unsigned)rb, (unsigned)ks), blk(64 * TK_WAVES);
      if (q8) {
        if (srt == 1) hipLaunchKernelGGL((gemm_s3_tall_kernel<1, true>), tg, blk, 0, c->stream, f, (float*)pt, spb);
        else if (srt == 2) hipLaunchKernelGGL((gemm_s3_tall_kernel<2, true>), tg, blk, 0, c->stream, f, (float*)pt, spb);
        else hipLaunchKernelGGL((gemm_s3_tall_kernel<3, true>), tg, blk, 0, c->stream, f, (float*)pt, spb);
      } else {
        if (srt == 1) hipLaunchKernelGGL((gemm_s3_tall_kernel<1, false>), tg, blk, 0, c->stream, f, (float*)pt, spb);
        else if (srt == 2) hipLaunchKernelGGL((gemm_s3_tall_kernel<2, false>), tg, blk, 0, c->stream, f, (float*)pt, spb);
        else hipLaunchKernelGGL((gemm_s3_tall_kernel<3, false>), tg, blk, 0, c->stream, f, (float*)pt, spb);
      }
      hipLaunchKernelGGL(s3_ksum_kernel, dim3((unsigned)(((M * N + 3) / 4 + 255) / 256)), dim3(256), 0, c->stream, f,
                         (const float*)pt, ks);
      anima_free(c, pt);
    }
    else if (N % 4 == 0 && ldc % 4 == 0 && al(d->out, 16) && (!W->bias || al(W->bias, 16)) &&
             (!d->add || (al(d->add, 16) && ld_add % 4 == 0)) &&
             (d->epilogue != ANIMA_EPI_GATED || al(d->gate + d->gate_off, 16)))
    {
      // four column tiles per wave where the grid stays large, one otherwise
      const int64_t big = (int64_t)((N + 255) / 256) * ((M + 63) / 64);
      if (big >= 1024)
        hipLaunchKernelGGL(gemm_s3_t_kernel<4>, dim3((N + 255) / 256, (unsigned)((M + 63) / 64)), dim3(256), 0, c->stream, f);
      else
        hipLaunchKernelGGL(gemm_s3_t_kernel<1>, dim3((N + 63) / 64, (unsigned)((M + 63) / 64)), dim3(256), 0, c->stream, f);
    }
    else
      return fail(c, ANIMA_E_ARG, "anima_linear: split weights with N > 256 need N %% 4 == 0 and 16-byte aligned out / bias / add / gate rows");
    return L.end();
  }
  if (W->kind == ANIMA_W_BF16 || W->kind == ANIMA_W_F32) {
    const bool f32 = W->kind == ANIMA_W_F32;
    if (!d->x) return fail(c, ANIMA_E_ARG, "anima_linear: bf16/fp32 weights need fp32 x");
    if (d->acc_out || d->xq) return fail(c, ANIMA_E_ARG, "anima_linear: acc_out / xq apply to i8/w4 weights only");
    const int64_t ldx = d->ldx ? d->ldx : K;
    if (ldx < K) return fail(c, ANIMA_E_ARG, "anima_linear: ldx < K");
    F32WArgs f{d->x, ldx, W->w, W->bias, d->out, ldc, alpha, d->act, d->epilogue, d->gate, d->gate_off,
               (int)M, N, K, 0, 0, 0, 0, d->add, ld_add, f32 ? 1 : 0};
    if (!f32 && M <= GEMV_MAXM && K % 8 == 0 && ldx % 4 == 0 && al(d->x, 16) && al(W->w, 16)) {
      Launch L(c, "gemv.bf16", 2.0 * M * N * K, 2.0 * N * K);
      hipLaunchKernelGGL(gemv_f32w_kernel, dim3((N + 3) / 4), dim3(256), 0, c->stream, f);
      return L.end();
    }
    const bool vec_out = N % 4 == 0 && ldc % 4 == 0 && al(d->out, 16) && (!W->bias || al(W->bias, 16)) &&
                         (!d->add || (al(d->add, 16) && ld_add % 4 == 0)) &&
                         (d->epilogue != ANIMA_EPI_GATED || al(d->gate + d->gate_off, 16));
    if (!f32 && N > 256 && K % 32 == 0 && M <= 65535LL * 32 && ldx % 4 == 0 && al(d->x, 16) && al(W->w, 16) && vec_out) {
      // bf16 matrix cores with x in three bf16 terms; k-groups per workgroup so that the grid
      // holds about 2048 waves while every k-group keeps at least 4 chunks
      Launch L(c, "gemm.bf16s3", 2.0 * M * N * K, 0.0);
      const int64_t ltiles = (int64_t)((N + 127) / 128) * ((M + 63) / 64);
      if (ltiles >= 128 && (M + 63) / 64 <= 65535) {  // wide grids: LDS-staged tiles
        hipLaunchKernelGGL(gemm_bf16_s3_lds_kernel, dim3((N + 127) / 128, (unsigned)((M + 63) / 64)), dim3(256), 0, c->stream, f);
        return L.end();
      }
      // small grids over long rows: k-slices of the LDS kernel into partial outputs, then one pass
      // that sums them and applies the epilogue
      int ks = 1;
      while (ks < 8 && ltiles * ks < 256 && (K / (2 * ks)) % 32 == 0 && K / (2 * ks) >= 256) ks *= 2;
      if (ks > 1 && (M + 63) / 64 <= 65535) {
        void* tmp = nullptr;
        int rc = anima_alloc(c, (size_t)ks * M * N * 4, &tmp);
        if (rc) return rc;
        F32WArgs g = f;
        g.out = (float*)tmp;
        g.ldc = N;
        g.alpha = 1.0f;
        g.bias = nullptr;
        g.add = nullptr;
        g.act = ANIMA_ACT_NONE;
        g.epi = ANIMA_EPI_STORE;
        g.K = K / ks;
        g.ldw = K;
        g.x_gs = K / ks;
        g.w_gs = K / ks;
        g.out_gs = (int64_t)M * N;
        hipLaunchKernelGGL(gemm_bf16_s3_lds_kernel, dim3((N + 127) / 128, (unsigned)((M + 63) / 64), ks), dim3(256), 0,
                           c->stream, g);
        const int64_t n_el = (int64_t)M * N;
        hipLaunchKernelGGL(splitk_epilogue_kernel, dim3((unsigned)((n_el + 255) / 256)), dim3(256), 0, c->stream,
                           (const float*)tmp, ks, f);
        anima_free(c, tmp);
        return L.end();
      }
      const int64_t tiles = (int64_t)((N + 127) / 128) * ((M + 31) / 32);
      const int nch = K / 32;
      int kgs = 1;
      while (kgs < 4 && tiles * 2 * kgs < 2048 && nch / (2 * kgs) >= 4) kgs *= 2;
      const dim3 grid((unsigned)((N + 127) / 128), (unsigned)((M + 31) / 32));
      if (kgs == 1) hipLaunchKernelGGL(gemm_bf16_s3_kernel<1>, grid, dim3(128), 0, c->stream, f);
      else if (kgs == 2) hipLaunchKernelGGL(gemm_bf16_s3_kernel<2>, grid, dim3(256), 0, c->stream, f);
      else hipLaunchKernelGGL(gemm_bf16_s3_kernel<4>, grid, dim3(512), 0, c->stream, f);
      return L.end();
    }
    Launch L(c, f32 ? "gemm.f32" : "gemm.bf16", 2.0 * M * N * K, 0.0);
    // fp32 matrix cores: x rows 16-byte aligned; weight rows 16-byte (fp32) / 8-byte (bf16) aligned
    if (K % 4 == 0 && ldx % 4 == 0 && al(d->x, 16) && al(W->w, f32 ? 16 : 8)) {
      const dim3 sk((unsigned)((N + 127) / 128), (unsigned)((M + 31) / 32)), blk(64 * SK_WAVES);
      const dim3 g64((N + 63) / 64, (unsigned)((M + 63) / 64));
      const bool vec = N % 4 == 0 && ldc % 4 == 0 && al(d->out, 16) && (!W->bias || al(W->bias, 16)) &&
                       (!d->add || (al(d->add, 16) && ld_add % 4 == 0)) &&
                       (d->epilogue != ANIMA_EPI_GATED || al(d->gate + d->gate_off, 16));
#define F32M_SKINNY(RT)                                                                  \
  do {                                                                                   \
    if (f32) hipLaunchKernelGGL((gemm_f32m_skinny_kernel<RT, false>), sk, blk, 0, c->stream, f); \
    else hipLaunchKernelGGL((gemm_f32m_skinny_kernel<RT, true>), sk, blk, 0, c->stream, f);      \
  } while (0)
      if (N <= 32 && K >= 512) F32M_SKINNY(1);
      else if (N <= 64 && K >= 512) F32M_SKINNY(2);
      else if (N <= 96 && K >= 512) F32M_SKINNY(3);
      else if (N <= 256 && K >= 512) F32M_SKINNY(4);
      else if (vec && f32) hipLaunchKernelGGL(gemm_f32m_t_kernel<false>, g64, dim3(256), 0, c->stream, f);
      else if (vec) hipLaunchKernelGGL(gemm_f32m_t_kernel<true>, g64, dim3(256), 0, c->stream, f);
      else if (f32) hipLaunchKernelGGL(gemm_f32m_kernel, g64, dim3(256), 0, c->stream, f);
      else hipLaunchKernelGGL(gemm_f32w_kernel, g64, dim3(256), 0, c->stream, f);
#undef F32M_SKINNY
      return L.end();
    }
    hipLaunchKernelGGL(gemm_f32w_kernel, dim3((N + 63) / 64, (unsigned)((M + 63) / 64)), dim3(256), 0, c->stream, f);
    return L.end();
  }
  if (W->kind != ANIMA_W_I8 && W->kind != ANIMA_W_W4) return fail(c, ANIMA_E_ARG, "anima_linear: unknown weight kind %d", W->kind);
  const bool w4 = W->kind == ANIMA_W_W4;
  if (K % GBK) return fail(c, ANIMA_E_ARG, "anima_linear: K=%d must be a multiple of %d for quantized weights", K, GBK);
  if (!W->scale || (w4 && (!W->srel || !W->codebook))) return fail(c, ANIMA_E_ARG, "anima_linear: missing scale/s_rel/codebook");
  if (!al(W->w, 16)) return fail(c, ANIMA_E_ARG, "anima_linear: weight data must be 16-byte aligned");

  const int8_t* qx = d->xq;
  const float* sx = d->xs;
  void* tmp = nullptr;
  if (!qx) {
    if (!d->x) return fail(c, ANIMA_E_ARG, "anima_linear: no input (x or xq)");
    const int64_t ldx = d->ldx ? d->ldx : K;
    if (ldx != K) return fail(c, ANIMA_E_ARG, "anima_linear: quantized weights need contiguous x (ldx == K)");
    if (K > 8192 || (!d->x_rotated && K % 256)) return fail(c, ANIMA_E_ARG, "anima_linear: K=%d (<= 8192, %% 256 == 0 to rotate)", K);
    int rc = anima_alloc(c, (size_t)M * K + (size_t)M * 4 + 256, &tmp);
    if (rc) return rc;
    int8_t* q = (int8_t*)tmp;
    float* s = (float*)((char*)tmp + ((size_t)M * K + 255) / 256 * 256);
    rc = quant_rows_launch(c, d->x, M, K, d->x_rotated ? 0 : 1, ANIMA_ACT_NONE, q, s);
    if (rc) {
      anima_free(c, tmp);
      return rc;
    }
    qx = q;
    sx = s;
  } else {
    if (!sx) return fail(c, ANIMA_E_ARG, "anima_linear: xq without xs");
    if (!al(qx, 16)) return fail(c, ANIMA_E_ARG, "anima_linear: xq must be 16-byte aligned");
  }
  GemmArgs g{qx, sx, W->w, W->scale, W->srel, W->codebook, W->bias, d->out, ldc, alpha, d->act, d->epilogue,
             d->gate, d->gate_off, d->acc_out, (int)M, N, K, d->add, ld_add};
  if (lora) {
    g.lx = d->lora_xa;
    g.ld_lx = d->ld_lora_xa;
    g.lb = d->lora_b;
    g.lr = d->lora_r;
    g.lcols = d->lora_cols;
  }
  int rc = ANIMA_OK;
  // Grids that give every CU a 256x256 tile run the persistent 256 kernel, smaller grids the
  // 128x128 kernel; both unpack W4 codes inside the GEMM.
  // The 256 kernel's epilogue moves 16-byte column groups: it needs N % 4 == 0 and 16-byte
  // aligned output rows, scales, bias and gate.
  const int64_t tiles256 = (int64_t)((N + 255) / 256) * ((M + 255) / 256);
  const bool vec = N % 4 == 0 && g.ldc % 4 == 0 && al(g.out, 16) && al(g.sw, 16) && (!g.bias || al(g.bias, 16)) &&
                   (g.epi != ANIMA_EPI_GATED || al(g.gate + g.gate_off, 16)) && (!g.add || (al(g.add, 16) && g.ld_add % 4 == 0));
  const bool big = vec && tiles256 >= c->num_cus && tiles256 <= 0x7fffffff;
  void* grid8 = nullptr;
  bool w4k = w4;  // the GEMM unpacks W4 codes itself
  // (a LoRA epilogue always runs on the int8 grid: the in-GEMM unpack leaves it no registers)
  if (big && w4 && (c->w4_path == ANIMA_W4_GRID_SCRATCH || lora)) {
    rc = w4_grid_scratch(c, W, g, &grid8);
    if (rc) {
      if (tmp) anima_free(c, tmp);
      return rc;
    }
    w4k = false;
  }
  // small grids, and rank blocks that split a 256-column tile: the LoRA product as an add term
  // (the split-bf16 kernel, one product per rank block over its columns' rows of the B planes)
  void* ldelta = nullptr;
  if (lora && (!big || d->lora_cols % 256)) {
    rc = anima_alloc(c, (size_t)M * N * 4, &ldelta);
    if (rc) {
      if (grid8) anima_free(c, grid8);
      if (tmp) anima_free(c, tmp);
      return rc;
    }
    const int bc = d->lora_cols ? d->lora_cols : N;
    for (int b = 0; b * bc < N && !rc; b++) {
      const anima_weight bw{ANIMA_W_F32S3, bc, d->lora_r, d->lora_b + (int64_t)b * bc * d->lora_r, nullptr, nullptr,
                            nullptr, nullptr};
      anima_linear_desc dd{};
      dd.M = M;
      dd.W = &bw;
      dd.x = d->lora_xa + (int64_t)b * d->lora_r;
      dd.ldx = d->ld_lora_xa;
      dd.out = (float*)ldelta + (int64_t)b * bc;
      dd.ldc = N;
      rc = linear_launch(c, &dd, (int64_t)N * d->lora_r);
    }
    g.add = (const float*)ldelta;
    g.ld_add = N;
    g.lr = 0;
  }
  if (!rc) {
    Launch L(c, w4k ? "gemm.w4a8" : "gemm.i8", 2.0 * M * N * K, 0.0);
    if (big) {
      const dim3 grid((unsigned)c->num_cus), block(512);
#define G2L(E, W)                                                                                    \
  {                                                                                                  \
    if (lora) hipLaunchKernelGGL((gemm_i8_256<E, false, false, true>), grid, block, 0, c->stream, g); \
    else hipLaunchKernelGGL((gemm_i8_256<E, W>), grid, block, 0, c->stream, g);                       \
  }
      if (g.epi == ANIMA_EPI_STORE) {
        if (w4k) G2L(ANIMA_EPI_STORE, true)
        else G2L(ANIMA_EPI_STORE, false)
      } else if (g.epi == ANIMA_EPI_RESID) {
        if (w4k) G2L(ANIMA_EPI_RESID, true)
        else G2L(ANIMA_EPI_RESID, false)
      } else {
        if (w4k) G2L(ANIMA_EPI_GATED, true)
        else G2L(ANIMA_EPI_GATED, false)
      }
#undef G2L
    } else {
      dim3 grid((N + GBN - 1) / GBN, (unsigned)((M + GBM - 1) / GBM));
      if (w4) hipLaunchKernelGGL(gemm_i8_kernel<true>, grid, dim3(256), 0, c->stream, g);
      else hipLaunchKernelGGL(gemm_i8_kernel<false>, grid, dim3(256), 0, c->stream, g);
    }
    rc = L.end();
  }
  if (ldelta) anima_free(c, ldelta);
  if (grid8) anima_free(c, grid8);
  if (tmp) anima_free(c, tmp);
  return rc;
}

// The stacked QKV projection with the attention operand epilogue (anima_linear_qkv).
int linear_qkv_launch(anima_ctx* c, const anima_linear_desc* d, const anima_qkv_desc* p) {
  if (!d || !p) return fail(c, ANIMA_E_ARG, "anima_linear_qkv: null descriptor");
  const anima_weight* W = d->W;
  if (!W) return fail(c, ANIMA_E_ARG, "anima_linear_qkv: null weight");
  if (W->kind != ANIMA_W_I8 && W->kind != ANIMA_W_W4)
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_linear_qkv: int8 or W4 weights only (kind %d)", W->kind);
  const int64_t M = d->M;
  const int N = W->N, K = W->K, H = p->H;
  if (p->B < 1 || p->L < 1 || H < 2 || H % 2 || (int64_t)p->B * p->L != M || M > 0x7fffffff)
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: B=%d L=%d H=%d M=%lld (M = B * L, H even)", p->B, p->L, H, (long long)M);
  if (p->L % 64) return fail(c, ANIMA_E_UNSUPPORTED, "anima_linear_qkv: L=%d must be a multiple of 64", p->L);
  const bool qonly = p->q_prep && N == H * HD_K;  // a Q-only projection (no K / V)
  if ((N != 3 * H * HD_K && !qonly) || K % GBK)
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: N=%d must be 3 * H * 128 = %d (or H * 128 with q_prep), K %% %d == 0", N,
                3 * H * HD_K, GBK);
  if (d->epilogue != ANIMA_EPI_STORE || d->act != ANIMA_ACT_NONE || d->add || d->acc_out)
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_linear_qkv: plain store only (no activation, residual, gate, add term or acc_out)");
  const bool lora = d->lora_xa || d->lora_b || d->lora_r;
  if (lora) {
    if (!d->lora_xa || !d->lora_b || d->lora_r < 16 || d->lora_r % 16 || d->ld_lora_xa % 4 || !al(d->lora_xa, 16) ||
        !al(d->lora_b, 16) || d->lora_cols < 0 || (d->lora_cols && (N % d->lora_cols || d->lora_cols % 256)) ||
        d->ld_lora_xa < (int64_t)d->lora_r * (d->lora_cols ? N / d->lora_cols : 1))
      return fail(c, ANIMA_E_ARG, "anima_linear_qkv: LoRA factors need lora_r %% 16 == 0 (%d), lora_cols 0 or a divisor of N "
                  "that is a multiple of 256 (%d), ld_lora_xa %% 4 == 0 covering the ranks (%lld), 16-byte aligned",
                  d->lora_r, d->lora_cols, (long long)d->ld_lora_xa);
  }
  if (!qonly && (!p->k_norm || !p->rope_cs || !p->kv_prep))
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: k_norm, rope_cs and kv_prep are required");
  if (!qonly && p->kv_prep_bytes != attention_kv_bytes(p->B, H, p->L, ANIMA_PREC_BF16))
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: kv_prep_bytes=%lld, the layout takes %lld", (long long)p->kv_prep_bytes,
                (long long)attention_kv_bytes(p->B, H, p->L, ANIMA_PREC_BF16));
  if (p->rope_cs) {
    const int64_t rows = p->rope_sin_off / (HD_K / 2);
    if (p->rope_sin_off <= 0 || p->rope_sin_off % (HD_K / 2) || rows < p->L)
      return fail(c, ANIMA_E_ARG, "anima_linear_qkv: rope_sin_off=%lld must be rows*64 with rows >= L=%d", (long long)p->rope_sin_off, p->L);
  }
  if ((p->q_prep && !al(p->q_prep, 16)) || (p->q_norm && !al(p->q_norm, 16)) || (p->rope_cs && !al(p->rope_cs, 16)))
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: q_prep, q_norm and rope_cs must be 16-byte aligned");
  const int64_t ldc = d->ldc ? d->ldc : N;
  if (!p->q_prep && (!d->out || ldc < H * HD_K))
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: out with ldc >= %d (the Q columns) required", H * HD_K);
  if (!W->w || !W->scale || (W->kind == ANIMA_W_W4 && (!W->srel || !W->codebook)))
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: missing weight data, scale, s_rel or codebook");
  if (!al(W->w, 16) || !al(d->out, 16) || ldc % 4 || !al(W->scale, 16) || (W->bias && !al(W->bias, 16)) ||
      !al(p->kv_prep, 16) || !al(p->k_norm, 16))
    return fail(c, ANIMA_E_ARG, "anima_linear_qkv: weight, out (ldc %% 4), scale, bias, kv_prep, k_norm and rope_cs must be 16-byte aligned");
  const int8_t* qx = d->xq;
  const float* sx = d->xs;
  void* tmp = nullptr;
  if (!qx) {
    if (!d->x) return fail(c, ANIMA_E_ARG, "anima_linear_qkv: no input (x or xq)");
    const int64_t ldx = d->ldx ? d->ldx : K;
    if (ldx != K) return fail(c, ANIMA_E_ARG, "anima_linear_qkv: contiguous x (ldx == K) required");
    if (K > 8192 || (!d->x_rotated && K % 256)) return fail(c, ANIMA_E_ARG, "anima_linear_qkv: K=%d (<= 8192, %% 256 == 0 to rotate)", K);
    int rc = anima_alloc(c, (size_t)M * K + (size_t)M * 4 + 256, &tmp);
    if (rc) return rc;
    int8_t* q = (int8_t*)tmp;
    float* s = (float*)((char*)tmp + ((size_t)M * K + 255) / 256 * 256);
    rc = quant_rows_launch(c, d->x, M, K, d->x_rotated ? 0 : 1, ANIMA_ACT_NONE, q, s);
    if (rc) {
      anima_free(c, tmp);
      return rc;
    }
    qx = q;
    sx = s;
  } else {
    if (!sx) return fail(c, ANIMA_E_ARG, "anima_linear_qkv: xq without xs");
    if (!al(qx, 16)) return fail(c, ANIMA_E_ARG, "anima_linear_qkv: xq must be 16-byte aligned");
  }
  const float alpha = d->alpha != 0.0f ? d->alpha : 1.0f;
  GemmArgs g{qx, sx, W->w, W->scale, W->srel, W->codebook, W->bias, d->out, ldc, alpha, ANIMA_ACT_NONE, ANIMA_EPI_STORE,
             nullptr, 0, nullptr, (int)M, N, K, nullptr, 0};
  g.kv = p->kv_prep;
  g.kv_plane = p->kv_prep_bytes / 2;
  g.kn = p->k_norm;
  g.cs = p->rope_cs;
  g.sin_off = p->rope_sin_off;
  g.eps = p->eps;
  g.L = p->L;
  g.Lkp = p->L;
  g.H = H;
  g.kcol = qonly ? N : H * HD_K;
  g.vcol = qonly ? N : 2 * H * HD_K;
  if (p->q_prep) {
    g.qn = p->q_norm;
    g.qp = (uint16_t*)p->q_prep;
    g.qc = (p->q_scale != 0.0f ? p->q_scale : 1.0f / sqrtf((float)HD_K)) * 1.4426950408889634f;
    g.qrope = p->rope_cs != nullptr;
  }
  if (lora) {
    g.lx = d->lora_xa;
    g.ld_lx = d->ld_lora_xa;
    g.lb = d->lora_b;
    g.lr = d->lora_r;
    g.lcols = d->lora_cols;
  }
  bool w4 = W->kind == ANIMA_W_W4;
  void* grid8 = nullptr;
  int rc;
  // (the LoRA epilogue always runs on the int8 grid: the in-GEMM unpack leaves it no registers)
  if (w4 && (c->w4_path == ANIMA_W4_GRID_SCRATCH || lora)) {
    rc = w4_grid_scratch(c, W, g, &grid8);
    if (rc) {
      if (tmp) anima_free(c, tmp);
      return rc;
    }
    w4 = false;
  }
  {
    Launch L(c, w4 ? "gemm.w4a8_qkv" : "gemm.i8_qkv", 2.0 * M * N * K, 0.0);
    // persistent 256 x 256 tiles (a tile holds two whole heads); one workgroup per CU at most
    const int64_t tiles = (int64_t)(N / 256) * ((M + 255) / 256);
    const dim3 grid((unsigned)(tiles < c->num_cus ? tiles : c->num_cus)), block(512);
    // (the prepared-Q epilogue is an instance of its own: its code raises the register pressure of
    // the main loop it shares the kernel with)
    if (lora && g.qp) hipLaunchKernelGGL((gemm_i8_256<ANIMA_EPI_STORE, false, true, true, true>), grid, block, 0, c->stream, g);
    else if (lora) hipLaunchKernelGGL((gemm_i8_256<ANIMA_EPI_STORE, false, true, true>), grid, block, 0, c->stream, g);
    else if (g.qp && w4) hipLaunchKernelGGL((gemm_i8_256<ANIMA_EPI_STORE, true, true, false, true>), grid, block, 0, c->stream, g);
    else if (g.qp) hipLaunchKernelGGL((gemm_i8_256<ANIMA_EPI_STORE, false, true, false, true>), grid, block, 0, c->stream, g);
    else if (w4) hipLaunchKernelGGL((gemm_i8_256<ANIMA_EPI_STORE, true, true>), grid, block, 0, c->stream, g);
    else hipLaunchKernelGGL((gemm_i8_256<ANIMA_EPI_STORE, false, true>), grid, block, 0, c->stream, g);
    rc = L.end();
  }
  if (grid8) anima_free(c, grid8);
  if (tmp) anima_free(c, tmp);
  return rc;
}

int linear_grouped_bf16_launch(anima_ctx* c, int G, int64_t M, int N, int K, const float* x, int64_t ldx,
                               int64_t x_gs, const uint16_t* w, int64_t w_gs, const float* bias, int64_t bias_gs,
                               float* out, int64_t ldc, int64_t out_gs) {
  if (!x || !w || !out) return fail(c, ANIMA_E_ARG, "anima_linear_grouped_bf16: null x, w or out");
  if (G < 1 || G > 65535 || M < 1 || M > GEMV_MAXM || N < 1 || K < 8 || K % 8)
    return fail(c, ANIMA_E_ARG, "anima_linear_grouped_bf16: G=%d M=%lld N=%d K=%d (1 <= G <= 65535, 1 <= M <= %d, K %% 8 == 0)",
                G, (long long)M, N, K, GEMV_MAXM);
  if (ldx < K || ldc < N || x_gs < 0 || w_gs < 0 || bias_gs < 0 || out_gs < 0)
    return fail(c, ANIMA_E_ARG, "anima_linear_grouped_bf16: bad leading dimension or group stride");
  if (!al(x, 16) || !al(w, 16) || ldx % 4 || x_gs % 4 || w_gs % 8)
    return fail(c, ANIMA_E_ARG, "anima_linear_grouped_bf16: x and w must be 16-byte aligned (ldx, x stride %% 4, w stride %% 8)");
  F32WArgs f{x, ldx, w, bias, out, ldc, 1.0f, ANIMA_ACT_NONE, ANIMA_EPI_STORE, nullptr, 0, (int)M, N, K,
             x_gs, w_gs, bias_gs, out_gs, nullptr, 0, 0};
  Launch L(c, "gemv.bf16.grouped", 2.0 * G * M * N * K, 2.0 * G * N * K);
  hipLaunchKernelGGL(gemv_f32w_kernel, dim3((N + 3) / 4, (unsigned)G), dim3(256), 0, c->stream, f);
  return L.end();
}

// G fp32 GEMVs, one output per thread: y_g[n] = alpha * sum_k w_g[n][k] x_g[k] (+ y_g[n]), the sum
// in k order with fp32 FMAs, the product then scaled and added as in the linear epilogues.
__global__ __launch_bounds__(256) void gemv_grouped_f32_kernel(const float* x, int64_t x_gs, const float* w, int64_t w_gs,
                                                               float* y, int64_t y_gs, int N, int K, float alpha,
                                                               int accumulate) {
  const int g = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const float4* wr = (const float4*)(w + g * w_gs + (int64_t)n * K);
  const float4* xr = (const float4*)(x + g * x_gs);
  float s = 0.0f;
  for (int k = 0; k < K / 4; k++) {
    const float4 a = wr[k], b = xr[k];
    s = __builtin_fmaf(a.x, b.x, s);
    s = __builtin_fmaf(a.y, b.y, s);
    s = __builtin_fmaf(a.z, b.z, s);
    s = __builtin_fmaf(a.w, b.w, s);
  }
  float* o = y + g * y_gs + n;
  const float r = s * alpha;
  *o = accumulate ? *o + r : r;
}

int gemv_grouped_f32_launch(anima_ctx* c, int G, int N, int K, const float* x, int64_t x_gs, const float* w, int64_t w_gs,
                            float* y, int64_t y_gs, float alpha, int accumulate) {
  if (!x || !w || !y) return fail(c, ANIMA_E_ARG, "anima_gemv_grouped_f32: null x, w or y");
  if (G < 1 || G > 65535 || N < 1 || K < 4 || K % 4)
    return fail(c, ANIMA_E_ARG, "anima_gemv_grouped_f32: G=%d N=%d K=%d (1 <= G <= 65535, K %% 4 == 0)", G, N, K);
  if (x_gs < 0 || w_gs < 0 || y_gs < 0 || x_gs % 4 || w_gs % 4 || !al(x, 16) || !al(w, 16))
    return fail(c, ANIMA_E_ARG, "anima_gemv_grouped_f32: x and w 16-byte aligned, x / w group strides >= 0 and %% 4 == 0");
  Launch L(c, "gemv.f32.grouped", 2.0 * G * N * K, 4.0 * G * N * K);
  hipLaunchKernelGGL(gemv_grouped_f32_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)G), dim3(256), 0, c->stream, x,
                     x_gs, w, w_gs, y, y_gs, N, K, alpha != 0.0f ? alpha : 1.0f, accumulate ? 1 : 0);
  return L.end();
}

}  // namespace anima

namespace anima {
int split3_launch(anima_ctx* c, const float* src, uint16_t* dst, int64_t n) {
  if (!src || !dst || n < 0 || n % 8) return fail(c, ANIMA_E_ARG, "anima_split3_bf16: n=%lld (n %% 8 == 0) or null pointer", (long long)n);
  if (!al(src, 16) || !al(dst, 16)) return fail(c, ANIMA_E_ARG, "anima_split3_bf16: pointers must be 16-byte aligned");
  if (n == 0) return ANIMA_OK;
  Launch L(c, "split3", 0.0, (double)n * 10);
  const int64_t n8 = n / 8, blocks = (n8 + 255) / 256;
  hipLaunchKernelGGL(split3_kernel, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, c->stream, src, dst, n8, n);
  return L.end();
}
}  // namespace anima
