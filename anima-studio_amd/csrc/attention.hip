// Fused DiT attention for gfx950: ops.attention's flash path (app/gpu/kernels.js:158-299) with
// the q/k RMSNorm + RoPE of qkNormRopeShader (kernels.js:304-334) folded in.
//
// Two kernels per call:
//   attn_prep_kv  K rows: optional RMSNorm + RoPE, rounded to the MFMA operand type and laid
//                 out [B][Hkv][Lkp][128]; V transposed to [B][Hkv][128][Lkp] so the P.V MFMA
//                 reads 4 consecutive keys per 8-byte LDS load.  Rows Lk..Lkp are zero.
//                 One pass over K and V (HBM-bound) instead of re-normalizing K in every
//                 query tile (32x redundant VALU work at N=4096).  bf16 operands take
//                 attn_prep_kv_lines (whole-line loads and stores, no LDS); fp32 operands the
//                 LDS-transpose kernel attn_prep_kv.
//   attn_flash_*  One workgroup = 4 waves x 32 queries.  Q is loaded from the fp32 input with
//                 RMSNorm + RoPE fused into the load and kept in registers; K/V tiles of 64
//                 keys stream through double-buffered LDS.  Scores are computed transposed,
//                 S^T = K Q^T, so every per-query quantity (running max, sum, rescale) is a
//                 per-lane scalar: lane (q, half) of a 32x32 MFMA tile owns query q.
//
// MFMA layouts used (32x32 tiles, 64 lanes, lane = n + 32*g):
//   A operand: lane (m + 32 g) supplies row m, k-group g;  B operand: lane (n + 32 g) supplies
//   column n, k-group g (the same per-register k order as A);  accumulator register r of lane
//   (n + 32 g) holds row 8*(r/4) + 4*g + (r%4), column n.
// Softmax uses exp2 and an integer running offset m.  The bf16 kernel rounds Q*c (c =
// scale*log2(e)) to bf16 and starts the S accumulators at -m, so p = exp2(S) directly; it has
// no per-block maximum (an overflow check on the row sums replaces it) and normalizes by the
// sum of the bf16-rounded p (the weights the P.V MFMA actually uses).  The fp32 kernel uses
// p = exp2(fma(s, c, -m)), raises m when a block maximum exceeds it by more than 8, and
// normalizes by the sum of p.  Integer offsets make the rounding of p independent of when
// the offset was raised (a power-of-two rescale).
#include <algorithm>
#include <cmath>
#include <mutex>

#include "common.h"
#include "internal.h"

namespace anima {

constexpr int HD = 128;        // head dim
constexpr int BQ = 128;        // queries per workgroup (4 waves x 32)
constexpr int BK = 64;         // keys per block
constexpr int MAXB = 64;       // max batch handled by one launch (kv_len in kernel args)
constexpr float RESCALE_SLACK = 8.0f;

struct PrepArgs {
  const float* k;
  int64_t ldk, k_bs;
  const float* v;
  int64_t ldv, v_bs;
  void* kb;  // [B][Hkv][Lkp][HD]
  void* vt;  // [B][Hkv][HD][Lkp]
  const float* kn;
  const float* cs;
  int64_t sin_off;
  float eps;
  int Hkv, Lk, Lkp;
  int D;  // the caller's head dim, 128 or 64 (dims D..127 of the operands are zero)
};

template <typename T>
__device__ __forceinline__ T cvt(float x);
template <>
__device__ __forceinline__ bf16 cvt<bf16>(float x) { return (bf16)x; }
template <>
__device__ __forceinline__ float cvt<float>(float x) { return x; }

// grid (Hkv, Lkp/64, B), 256 threads.  Every thread issues all of its K and V loads first (one
// memory round trip per workgroup instead of one for K and then one for V).
template <typename T, bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void attn_prep_kv(PrepArgs a) {
  constexpr int VSP = BK + (sizeof(T) == 2 ? 2 : 4);  // padded LDS row (keys) of the V transpose
  __shared__ T vs[HD * VSP];
  const int t = threadIdx.x;
  const int kb0 = blockIdx.y * BK, hk = blockIdx.x, b = blockIdx.z;
  const int64_t head_row0 = ((int64_t)b * a.Hkv + hk) * a.Lkp;

  // V rows of this thread: dim group g -> dims 8g..8g+7, token group tg -> tokens 4tg..4tg+3
  const int g = (t & 7) | (((t >> 5) & 1) << 3), tg = ((t >> 3) & 3) | ((t >> 6) << 2);
  // Loads are unconditional (rows past Lk read row Lk-1, then count as zero), so they issue
  // back to back instead of one branch (and one wait) per row.
  float e[4][8];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int l = kb0 + 4 * tg + j;
    const float* src = a.v + (int64_t)b * a.v_bs + (int64_t)min(l, a.Lk - 1) * a.ldv + hk * a.D + 8 * g;
    const bool in = 8 * g < a.D;  // D = 64: dim groups 8..15 are padding
    const float4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    const float4 lo = in ? *(const float4*)src : z, hi = in ? *(const float4*)(src + 4) : z;
    e[j][0] = lo.x; e[j][1] = lo.y; e[j][2] = lo.z; e[j][3] = lo.w;
    e[j][4] = hi.x; e[j][5] = hi.y; e[j][6] = hi.z; e[j][7] = hi.w;
  }

  // ---- K: thread = (row t/4, quarter t%4); quarter p owns dims [16p,16p+16) and +64.  The row,
  // its norm weights and its RoPE table entries are loaded here too, then a scheduling fence
  // keeps every load of the thread ahead of the first wait.
  {
    const int r = t >> 2, p = t & 3, l = kb0 + r;
    float x[32], w[32], cv[16], sv[16];
    {
      const float* src = a.k + (int64_t)b * a.k_bs + (int64_t)min(l, a.Lk - 1) * a.ldk + hk * a.D;
      const bool hi = a.D == HD;  // D = 64: dims 64..127 are padding
#pragma unroll
      for (int j = 0; j < 4; j++) {
        *(float4*)(x + 4 * j) = *(const float4*)(src + 16 * p + 4 * j);
        *(float4*)(x + 16 + 4 * j) = hi ? *(const float4*)(src + 64 + 16 * p + 4 * j) : (float4){0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
    if (NORM) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        *(float4*)(w + 4 * j) = *(const float4*)(a.kn + 16 * p + 4 * j);
        *(float4*)(w + 16 + 4 * j) = *(const float4*)(a.kn + 64 + 16 * p + 4 * j);
      }
    }
    if (ROPE) {
      const float* cr = a.cs + (int64_t)min(l, a.Lk - 1) * (HD / 2) + 16 * p;  // rows of 64, 16-byte aligned
#pragma unroll
      for (int j = 0; j < 4; j++) {
        *(float4*)(cv + 4 * j) = *(const float4*)(cr + 4 * j);
        *(float4*)(sv + 4 * j) = *(const float4*)(cr + a.sin_off + 4 * j);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (l >= a.Lk) {
#pragma unroll
      for (int i = 0; i < 32; i++) x[i] = 0.0f;
    }
    if (NORM) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; i++) ss += x[i] * x[i];
      ss += __shfl_xor(ss, 1);
      ss += __shfl_xor(ss, 2);
      const float rn = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
      for (int i = 0; i < 16; i++) {
        x[i] = x[i] * rn * w[i];
        x[16 + i] = x[16 + i] * rn * w[16 + i];
      }
    }
    if (ROPE && l < a.Lk) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float c = cv[i], s = sv[i];
        const float x1 = x[i], x2 = x[16 + i];
        x[i] = x1 * c - x2 * s;
        x[16 + i] = x2 * c + x1 * s;
      }
    }
    T* dst = (T*)a.kb + (head_row0 + l) * HD;
    if constexpr (sizeof(T) == 2) {
      bf16x8 o[4];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        o[0][i] = to_bf16(x[i]);
        o[1][i] = to_bf16(x[8 + i]);
        o[2][i] = to_bf16(x[16 + i]);
        o[3][i] = to_bf16(x[24 + i]);
      }
      *(bf16x8*)(dst + 16 * p) = o[0];
      *(bf16x8*)(dst + 16 * p + 8) = o[1];
      *(bf16x8*)(dst + 64 + 16 * p) = o[2];
      *(bf16x8*)(dst + 64 + 16 * p + 8) = o[3];
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        *(float4*)((float*)dst + 16 * p + 4 * j) = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
        *(float4*)((float*)dst + 64 + 16 * p + 4 * j) =
            make_float4(x[16 + 4 * j], x[16 + 4 * j + 1], x[16 + 4 * j + 2], x[16 + 4 * j + 3]);
      }
    }
  }

  // ---- V (loaded above): each half-wave holds dim groups 0-7 or 8-15 and four token groups, so
  // with the 66-element LDS rows its 8-byte writes (four tokens of one dim) cover all 64 banks
  // once.
  {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (kb0 + 4 * tg + j >= a.Lk) {
#pragma unroll
        for (int i = 0; i < 8; i++) e[j][i] = 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      T* row = vs + (8 * g + i) * VSP + 4 * tg;
#pragma unroll
      for (int j = 0; j < 4; j++) row[j] = cvt<T>(e[j][i]);
    }
    __syncthreads();
    // write rows of V^T: thread = (dim t/2, half t%2 -> 32 keys)
    const int d = t >> 1, h2 = t & 1;
    T* dst = (T*)a.vt + (((int64_t)b * a.Hkv + hk) * HD + d) * a.Lkp + kb0 + 32 * h2;
    const T* srow = vs + d * VSP + 32 * h2;
    if constexpr (sizeof(T) == 2) {
      // bf16 MFMA layout: each 16-key group stored as keys [0-3, 8-11, 4-7, 12-15]
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int g16 = (i >> 1) * 16, half = i & 1;
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          o[e] = ((const bf16*)srow)[g16 + 4 * half + e];
          o[4 + e] = ((const bf16*)srow)[g16 + 8 + 4 * half + e];
        }
        *(bf16x8*)((bf16*)dst + 8 * i) = o;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float* s4 = (const float*)srow + 4 * i;
        *(float4*)((float*)dst + 4 * i) = make_float4(s4[0], s4[1], s4[2], s4[3]);
      }
    }
  }
}

// bf16 K / V prep with whole-line accesses: every load and store instruction of a wave moves
// complete 128-byte lines, and no LDS is used.  grid (Hkv, Lkp/64, B), 256 threads; one
// workgroup = one kv head x 64 keys of one batch element.
//   K: 16 lanes per key row, lane q holding dims 4q..4q+3 and 64+4q..64+4q+3 (so each RoPE pair is
//      in one lane); wave w takes rows 16w .. 16w+15, four per load instruction.  The row's sum of
//      squares crosses its 16 lanes by lane shuffles in a fixed tree.
//   V: wave w takes dims 32w .. 32w+31 of all 64 keys; lane (q = lane % 8, c = lane / 8) loads the
//      8 keys of V^T chunk c (the MFMA key order: each 16-key group stored as keys 0-3, 8-11, 4-7,
//      12-15) at dims 32w+4q .. +3 and stores four 16-byte chunks, one per dim; the 8 lanes of one
//      dim cover its 64 keys (128 bytes).
template <bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void attn_prep_kv_lines(PrepArgs a) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  // key blocks fastest: consecutive workgroups write consecutive 128-byte pieces of the same V^T
  // rows (and consecutive K rows)
  const int kb0 = blockIdx.x * BK, hk = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * a.Hkv + hk;
  // ---- all loads first
  const int q16 = lane & 15, rsub = lane >> 4;
  float4 klo[4], khi[4], cv[4], sv[4], wl = {}, wh = {};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int l = min(kb0 + 16 * w + 4 * i + rsub, a.Lk - 1);
    const float* src = a.k + (int64_t)b * a.k_bs + (int64_t)l * a.ldk + hk * a.D + 4 * q16;
    klo[i] = *(const float4*)src;
    khi[i] = a.D == HD ? *(const float4*)(src + 64) : (float4){0.0f, 0.0f, 0.0f, 0.0f};  // D = 64: padding
    if (ROPE) {
      const float* cr = a.cs + (int64_t)l * (HD / 2) + 4 * q16;
      cv[i] = *(const float4*)cr;
      sv[i] = *(const float4*)(cr + a.sin_off);
    }
  }
  if (NORM) {
    wl = *(const float4*)(a.kn + 4 * q16);
    wh = *(const float4*)(a.kn + 64 + 4 * q16);
  }
  const int vq = lane & 7, vc = lane >> 3;
  float4 ve[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int key = kb0 + 16 * (vc >> 1) + 4 * (vc & 1) + (e & 3) + 8 * (e >> 2);
    ve[e] = 32 * w < a.D ? *(const float4*)(a.v + (int64_t)b * a.v_bs + (int64_t)min(key, a.Lk - 1) * a.ldv + hk * a.D + 32 * w + 4 * vq)
                         : (float4){0.0f, 0.0f, 0.0f, 0.0f};  // D = 64: waves 2, 3 write the zero dims
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- K rows
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int l = kb0 + 16 * w + 4 * i + rsub;
    float x[8] = {klo[i].x, klo[i].y, klo[i].z, klo[i].w, khi[i].x, khi[i].y, khi[i].z, khi[i].w};
    if (NORM) {
      // The sum of squares over the row's 128 dims in a fixed tree (the QKV GEMM's attention
      // operand epilogue, anima_linear_qkv, forms the same one): this lane's 8 squares chained
      // by fma, then its partners across lane bits 1 and 2 (pairs of 8-dim leaves), bit 0 (the
      // two 4-dim halves of each 8) and bit 3 (the two 32-dim groups of each 64).
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; j++) ss = __builtin_fmaf(x[j], x[j], ss);
      ss = ss + __shfl_xor(ss, 2);
      ss = ss + __shfl_xor(ss, 4);
      ss = ss + __shfl_xor(ss, 1);
      ss = ss + __shfl_xor(ss, 8);
      const float rn = 1.0f / sqrtf(__builtin_fmaf(ss, 1.0f / (float)HD, a.eps));
      const float wv[8] = {wl.x, wl.y, wl.z, wl.w, wh.x, wh.y, wh.z, wh.w};
#pragma unroll
      for (int j = 0; j < 8; j++) x[j] = (x[j] * rn) * wv[j];
    }
    if (ROPE) {
      const float c4[4] = {cv[i].x, cv[i].y, cv[i].z, cv[i].w}, s4[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float x1 = x[j], x2 = x[4 + j];
        x[j] = __builtin_fmaf(x1, c4[j], -(x2 * s4[j]));
        x[4 + j] = __builtin_fmaf(x2, c4[j], x1 * s4[j]);
      }
    }
    bf16x4 lo, hi;
    const bool live = l < a.Lk;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      lo[j] = to_bf16(live ? x[j] : 0.0f);
      hi[j] = to_bf16(live ? x[4 + j] : 0.0f);
    }
    // (non-temporal stores: the operands are read back by the flash kernel, from HBM either way)
    bf16* dst = (bf16*)a.kb + (bh * a.Lkp + l) * HD + 4 * q16;
    __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, lo), (uint64_t*)dst);
    __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, hi), (uint64_t*)(dst + 64));
  }
  // ---- V^T chunks
  bf16* vdst = (bf16*)a.vt + (bh * HD + 32 * w + 4 * vq) * a.Lkp + kb0 + 8 * vc;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int key = kb0 + 16 * (vc >> 1) + 4 * (vc & 1) + (e & 3) + 8 * (e >> 2);
      const float v = j == 0 ? ve[e].x : j == 1 ? ve[e].y : j == 2 ? ve[e].z : ve[e].w;
      o[e] = to_bf16(key < a.Lk ? v : 0.0f);
    }
    uint64_t* q = (uint64_t*)(vdst + (int64_t)j * a.Lkp);
    __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, (bf16x4){o[0], o[1], o[2], o[3]}), q);
    __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, (bf16x4){o[4], o[5], o[6], o[7]}), q + 1);
  }
}

struct FlashArgs {
  const float* q;
  int64_t ldq, q_bs;
  const void* kb;
  const void* vt;
  float* o;
  int64_t ldo, o_bs;
  const float* qn;
  const float* cs;
  int64_t sin_off;
  float eps, c;  // c = scale * log2(e)
  int H, group, Hkv, Lq, Lkp, n_qt;
  int kv_len[MAXB];
  int causal;  // keys > query index masked (the 4-wave and fp32 kernels)
  int D;       // the caller's head dim, 128 or 64 (the operands are zero-padded to 128)
  // prepared Q (the bf16 kernels' QP form): [B][Lq][H][128] bf16, each value the kernel's own
  // to_bf16(c * q') of the normed, rotated query q'; then q, qn and cs are not read
  const uint16_t* qp;
  int obf;  // O written as bf16 (o then addresses uint16 elements)
};

// Loads this lane's 64 Q values (query qi, dims 16ks + 8hf + j), applies the fused
// RMSNorm + RoPE, and returns them in x[ks*8 + j].
template <bool NORM, bool ROPE>
__device__ __forceinline__ void q_post(const FlashArgs& a, int qi, int hf, float* x);
template <bool NORM>
__device__ __forceinline__ void q_norm(const FlashArgs& a, int hf, float* x);
__device__ __forceinline__ void q_rope(float* x, const float* c, const float* sn);

template <bool NORM, bool ROPE>
__device__ __forceinline__ void load_q(const FlashArgs& a, int b, int h, int qi, int hf, float* x) {
  if (qi < a.Lq) {
    const float* src = a.q + (int64_t)b * a.q_bs + (int64_t)qi * a.ldq + h * a.D + 8 * hf;
    const float4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      const bool in = 16 * ks < a.D;  // D = 64: k-steps 4..7 are padding
      float4 lo = in ? *(const float4*)(src + 16 * ks) : z;
      float4 hi = in ? *(const float4*)(src + 16 * ks + 4) : z;
      x[8 * ks] = lo.x; x[8 * ks + 1] = lo.y; x[8 * ks + 2] = lo.z; x[8 * ks + 3] = lo.w;
      x[8 * ks + 4] = hi.x; x[8 * ks + 5] = hi.y; x[8 * ks + 6] = hi.z; x[8 * ks + 7] = hi.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; i++) x[i] = 0.0f;
  }
  q_post<NORM, ROPE>(a, qi, hf, x);
}

// The q RMSNorm and RoPE of load_q on the lane's 64 values x[8 ks + j] (dims 16 ks + 8 hf + j):
// the sum of squares over the lane pair, then weights, then the split-half rotation.
template <bool NORM, bool ROPE>
__device__ __forceinline__ void q_post(const FlashArgs& a, int qi, int hf, float* x) {
  q_norm<NORM>(a, hf, x);
  if (ROPE && qi < a.Lq) {
    const float* cr = a.cs + (int64_t)qi * (HD / 2) + 8 * hf;
    const float* sr = a.cs + a.sin_off + (int64_t)qi * (HD / 2) + 8 * hf;
    float c[32], sn[32];
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        c[8 * ks + j] = cr[16 * ks + j];
        sn[8 * ks + j] = sr[16 * ks + j];
      }
    q_rope(x, c, sn);
  }
}

// The lane's split-half rotation with its cos / sin values c[8 ks + j], s[8 ks + j] (dims
// 16 ks + 8 hf + j of the table row).
__device__ __forceinline__ void q_rope(float* x, const float* c, const float* sn) {
#pragma unroll
  for (int ks = 0; ks < 4; ks++)
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float x1 = x[8 * ks + j], x2 = x[8 * (ks + 4) + j];
      // the rotation in the fused form of the K operand epilogue
      x[8 * ks + j] = __builtin_fmaf(x1, c[8 * ks + j], -(x2 * sn[8 * ks + j]));
      x[8 * (ks + 4) + j] = __builtin_fmaf(x2, c[8 * ks + j], x1 * sn[8 * ks + j]);
    }
}

template <bool NORM>
__device__ __forceinline__ void q_norm(const FlashArgs& a, int hf, float* x) {
  if (NORM) {
    // The row's sum of squares in one fixed tree, that of the K operand epilogue of the stacked
    // QKV projection (so a Q prepared there is bit-identical): leaves of 8 values, dims
    // 32 g + 8 q + 4 h + e then 64 + the same (e = 0..3, fused multiply-adds in that order); per
    // (g, h): (L0 + L1) + (L2 + L3) over q; then the two h; then the two g.  This lane holds the
    // leaves q = 2 qq + hf (dims 16 ks + 8 hf + j with ks = 2 g + qq, j = 4 h + e), its pair lane
    // the others.  (fp addition is commutative, so both lanes reach the same bits.)
    float part[2][2];
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float lf[2];
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
          const int ks = 2 * g + qq;
          float acc = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; e++) acc = __builtin_fmaf(x[8 * ks + 4 * h + e], x[8 * ks + 4 * h + e], acc);
#pragma unroll
          for (int e = 0; e < 4; e++) acc = __builtin_fmaf(x[8 * (ks + 4) + 4 * h + e], x[8 * (ks + 4) + 4 * h + e], acc);
          lf[qq] = acc;
        }
        const float o0 = __shfl_xor(lf[0], 32), o1 = __shfl_xor(lf[1], 32);
        part[g][h] = (lf[0] + o0) + (lf[1] + o1);
      }
    const float ss = (part[0][0] + part[0][1]) + (part[1][0] + part[1][1]);
    const float rn = 1.0f / sqrtf(__builtin_fmaf(ss, 1.0f / 128.0f, a.eps));
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int j = 0; j < 8; j++) x[8 * ks + j] = x[8 * ks + j] * rn * a.qn[16 * ks + 8 * hf + j];
  }
}

// ------------------------------------------------------------------ bf16 MFMA kernel

// LDS tiles of one stage for KB keys per block: K [KB][HD] rows of 272 B (conflict-free 16-byte
// fragment reads), V^T [HD][KB] rows of 2*KB + 16 B (16-byte aligned).
// max / sum of a value over the lane pair (l, l ^ 32) on the VALU: v_permlane32_swap exchanges
// the upper half of its first operand with the lower half of its second, so with both operands
// equal to x the two results hold x and its partner (in either order) in every lane.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int KB>
struct Tiles {
  static constexpr int KSP = HD + 8;
  static constexpr int VSP = KB + 8;
  static constexpr int KTILE = KB * KSP;
  static constexpr int STAGE = KTILE + HD * VSP;
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// LDS addressing of the K and V^T fragments a lane reads (tile t = 32 keys, k-step ks = 16 dims,
// dim tile dt = 32 dims, h = 16-key half of a key tile).
// Padded layout: K rows of KB keys x (128 + 8) bf16, V^T rows of 128 dims x (KB + 8) bf16.
template <int KB>
struct PadAddr {
  const bf16* kb;  // K + lq*KSP + 8hf
  const bf16* vb;  // V + lq*VSP + 8hf
  __device__ __forceinline__ PadAddr(const bf16* K, const bf16* V, int lq, int hf)
      : kb(K + lq * Tiles<KB>::KSP + 8 * hf), vb(V + lq * Tiles<KB>::VSP + 8 * hf) {}
  __device__ __forceinline__ bf16x8 k(int t, int ks) const {
    return *(const bf16x8*)(kb + t * 32 * Tiles<KB>::KSP + 16 * ks);
  }
  __device__ __forceinline__ bf16x8 v(int t, int dt, int h) const {
    return *(const bf16x8*)(vb + dt * 32 * Tiles<KB>::VSP + 32 * t + 16 * h);
  }
};

// Swizzled layout of 64-key blocks (direct-to-LDS copies cannot pad rows): K rows of 256 B whose
// 16-byte unit u sits at slot u ^ (row % 16); V^T rows of 128 B with unit u at u ^ ((row/2) % 8).
// Any 16 consecutive rows of either tile then map one unit index to 16 distinct bank groups.
constexpr int SWZ_KT = 64 * HD * 2;  // K tile bytes; the V^T tile follows
struct SwzOfs {
  int k[8], v[4];  // lane parts: k[ks] (row lq of key tile 0), v[2t+h] (row lq of dim tile 0)
  // base: a constant added to every part, so that a stage address can stay within the 16-bit
  // immediate offset of ds_read
  __device__ __forceinline__ SwzOfs(int lq, int hf, int base = 0) {
#pragma unroll
    for (int ks = 0; ks < 8; ks++) k[ks] = base + lq * 256 + 16 * ((2 * ks + hf) ^ (lq & 15));
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = base + SWZ_KT + lq * 128 + 16 * ((2 * j + hf) ^ ((lq >> 1) & 7));
  }
};
struct SwzAddr {
  const char* st;  // stage base
  const SwzOfs& of;
  __device__ __forceinline__ SwzAddr(const char* s, const SwzOfs& o) : st(s), of(o) {}
  __device__ __forceinline__ bf16x8 k(int t, int ks) const { return *(const bf16x8*)(st + of.k[ks] + t * 32 * 256); }
  __device__ __forceinline__ bf16x8 v(int t, int dt, int h) const {
    return *(const bf16x8*)(st + of.v[2 * t + h] + dt * 32 * 128);
  }
};

// One KB-key block for one wave of 32 queries.  Q arrives pre-scaled by c = scale*log2(e), and
// the running offset is folded into the accumulator init of S^T = K Q^T (srcC = -m), so the
// MFMA yields x = s*c - m directly and p = exp2(x) needs no other VALU work.
//
// The offset m is an integer that only moves up.  The first block sets it to ceil(block max);
// later blocks do not compute a maximum at all: the 16 probabilities a lane holds for one key
// tile are summed anyway (the row sum l), and that sum bounds each of them, so a tile whose
// lane sum stays <= 2^64 cannot have overflowed.  Only when a lane sum exceeds 2^64 (or is inf)
// the wave takes the rare path: raise m by ceil(max x) of that tile, rescale O and l by the
// exact power of two, and recompute the tile's probabilities.  Because m is an integer, the
// bf16 rounding of every p is independent of when m moved (an exact power-of-two scale), and
// the largest weight of the first block is >= 1/2, so l never underflows.
//
// Accumulator register r of key tile t holds key 32t + 8(r/4) + 4hf + r%4; P.V k-step s
// (16 keys) takes registers 8(s%2)..+7 of tile s/2, i.e. keys 16s + 8(j/4) + 4hf + j%4.  V^T
// rows hold each 16-key group as keys [0-3, 8-11, 4-7, 12-15], so the matching 8 keys of lane
// half hf are one 16-byte read.  The P.V product of tile t is issued right after its
// probabilities, so its MFMAs overlap the exponentials of tile t+1.
// MASK: keys >= Lk get -inf (last block only).  FIRST: the block that initializes m.
constexpr float P_LIMIT = 18446744073709551616.0f;  // 2^64

template <int KB, bool MASK, bool FIRST, class Addr>
__device__ __forceinline__ void flash_block(const Addr& A, const bf16x8 (&qf)[8], f32x16 (&o)[4], float& m,
                                            f32x16& negm, float& l, int key0, int Lk, int hf) {
  constexpr int NKT = KB / 32;
  f32x16 s[NKT];
#pragma unroll
  for (int t = 0; t < NKT; t++) {
    s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A.k(t, 0), qf[0], FIRST ? (f32x16){} : negm, 0, 0, 0);
#pragma unroll
    for (int ks = 1; ks < 8; ks++) s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A.k(t, ks), qf[ks], s[t], 0, 0, 0);
  }
  if (MASK) {
#pragma unroll
    for (int t = 0; t < NKT; t++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        if (key0 + 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3) >= Lk) s[t][r] = -INFINITY;
  }
  if (FIRST) {  // the first block holds at least one valid key of every query: bm is finite
    float bm = s[0][0];
#pragma unroll
    for (int t = 0; t < NKT; t++)
#pragma unroll
      for (int r = (t == 0 ? 1 : 0); r < 16; r++) bm = fmaxf(bm, s[t][r]);
    m = ceilf(pair_max(bm));
#pragma unroll
    for (int t = 0; t < NKT; t++) s[t] -= m;
    negm = -m;
  }
  const bf16x2 ones = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
  for (int t = 0; t < NKT; t++) {
    bf16x8 p0, p1;
    float l0 = 0.0f, l1 = 0.0f;
#define ANIMA_PROBS()                                                                                        \
  {                                                                                                          \
    _Pragma("unroll") for (int r = 0; r < 8; r++) {                                                          \
      p0[r] = to_bf16(__builtin_amdgcn_exp2f(s[t][r]));                                                      \
      p1[r] = to_bf16(__builtin_amdgcn_exp2f(s[t][8 + r]));                                                  \
    }                                                                                                        \
    l0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p0, p0, 0, 1), ones, 0.0f, false);          \
    l1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p0, p0, 2, 3), ones, 0.0f, false);          \
    l0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p0, p0, 4, 5), ones, l0, false);            \
    l1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p0, p0, 6, 7), ones, l1, false);            \
    l0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p1, p1, 0, 1), ones, l0, false);            \
    l1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p1, p1, 2, 3), ones, l1, false);            \
    l0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p1, p1, 4, 5), ones, l0, false);            \
    l1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p1, p1, 6, 7), ones, l1, false);            \
  }
    ANIMA_PROBS();
    if (!FIRST && __builtin_expect(__builtin_amdgcn_ballot_w64(!(l0 + l1 <= P_LIMIT)) != 0, 0)) {
      // rare: some probability of this tile exceeds 2^64; move the offset up to its maximum
      float bm = s[t][0];
#pragma unroll
      for (int r = 1; r < 16; r++) bm = fmaxf(bm, s[t][r]);
      const float d = fmaxf(ceilf(pair_max(bm)), 0.0f);
      const float alpha = __builtin_amdgcn_exp2f(-d);
      m += d;
      negm -= d;
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] *= alpha;
#pragma unroll
      for (int u = t; u < NKT; u++) s[u] -= d;
      ANIMA_PROBS();
    }
#undef ANIMA_PROBS
    l += l0 + l1;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
      o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A.v(t, dt, 0), p0, o[dt], 0, 0, 0);
      o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A.v(t, dt, 1), p1, o[dt], 0, 0, 0);
    }
  }
}

// Main-path block (64 keys, no mask, offset already set), hand-ordered: sched_barrier(0) fences
// keep the written order, so each MFMA finds its K / V^T fragment loaded four reads earlier and
// the exponentials of one key tile sit between the MFMAs of the next product.
#define ANIMA_SB() __builtin_amdgcn_sched_barrier(0)
// On entry f holds fragments 0..3 of block A; with NEXT, fragments 0..3 of block N (already
// published) are read during the last MFMAs and left in f, otherwise f is left undefined.
template <class Addr, bool NEXT>
__device__ __forceinline__ void flash_block_main(const Addr& A, const Addr& N, bf16x8 (&f)[4], const bf16x8 (&qf)[8],
                                                 f32x16 (&o)[4], float& m, f32x16& negm, float& l) {
  // fragment i of the block: K reads 0..15 (tile i/8, k-step i%8), V^T reads 16..31
  // (key tile (i-16)/8, dim tile ((i-16)%8)/2, 16-key half (i-16)%2)
#define FRAG(i) ((i) < 16 ? A.k((i) >> 3, (i) & 7) : A.v(((i) - 16) >> 3, (((i) - 16) & 7) >> 1, ((i) - 16) & 1))
  f32x16 s0, s1;
  bf16x8 p[4];  // p[0], p[1]: tile 0;  p[2], p[3]: tile 1
  const bf16x2 ones = {(bf16)1.0f, (bf16)1.0f};
  float la = 0.0f, lb = 0.0f;
  // 2 probabilities of tile T (registers 2k, 2k+1 of S) -> p, row-sum partial
#define PROB2(S, T, k)                                                                                \
  {                                                                                                   \
    bf16x8& pp_ = p[2 * (T) + ((k) >> 2)];                                                            \
    pp_[2 * ((k) & 3)] = to_bf16(__builtin_amdgcn_exp2f(S[2 * (k)]));                                 \
    pp_[2 * ((k) & 3) + 1] = to_bf16(__builtin_amdgcn_exp2f(S[2 * (k) + 1]));                         \
    float& acc_ = ((k) & 1) ? lb : la;                                                                \
    const bf16x2 pr_ = {pp_[2 * ((k) & 3)], pp_[2 * ((k) & 3) + 1]};                                 \
    acc_ = __builtin_amdgcn_fdot2_f32_bf16(pr_, ones, acc_, false);                                   \
  }
  // S tile 0: MFMAs 0..7, reads 4..11
#pragma unroll
  for (int i = 0; i < 8; i++) {
    s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i & 3], qf[i], i == 0 ? negm : s0, 0, 0, 0);
    f[i & 3] = FRAG(i + 4);
    ANIMA_SB();
  }
  // S tile 1: MFMAs 8..15, reads 12..19; tile-0 probabilities between them
#pragma unroll
  for (int i = 8; i < 16; i++) {
    s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i & 3], qf[i - 8], i == 8 ? negm : s1, 0, 0, 0);
    f[i & 3] = FRAG(i + 4);
    PROB2(s0, 0, i - 8);
    ANIMA_SB();
  }
  float lt = la + lb;
  if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(lt <= P_LIMIT)) != 0, 0)) {
    float bm = s0[0];
#pragma unroll
    for (int r = 1; r < 16; r++) bm = fmaxf(bm, s0[r]);
    const float d = fmaxf(ceilf(pair_max(bm)), 0.0f);
    const float alpha = __builtin_amdgcn_exp2f(-d);
    m += d;
    negm -= d;
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] *= alpha;
    s0 -= d;
    s1 -= d;
    la = lb = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) PROB2(s0, 0, k);
    lt = la + lb;
  }
  l += lt;
  la = lb = 0.0f;
  ANIMA_SB();
  // P.V tile 0: MFMAs 16..23 (fragments 16..23), reads 20..27; tile-1 probabilities
#pragma unroll
  for (int j = 0; j < 8; j++) {
    o[j >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[j & 3], p[j & 1], o[j >> 1], 0, 0, 0);
    f[j & 3] = FRAG(j + 20);
    PROB2(s1, 1, j);
    ANIMA_SB();
  }
  lt = la + lb;
  if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(lt <= P_LIMIT)) != 0, 0)) {
    float bm = s1[0];
#pragma unroll
    for (int r = 1; r < 16; r++) bm = fmaxf(bm, s1[r]);
    const float d = fmaxf(ceilf(pair_max(bm)), 0.0f);
    const float alpha = __builtin_amdgcn_exp2f(-d);
    m += d;
    negm -= d;
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] *= alpha;
    s1 -= d;
    la = lb = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) PROB2(s1, 1, k);
    lt = la + lb;
  }
  l += lt;
  ANIMA_SB();
  // P.V tile 1: MFMAs 24..31 (fragments 24..31), reads 28..31, then block N's 0..3
#pragma unroll
  for (int j = 0; j < 8; j++) {
    o[j >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[j & 3], p[2 + (j & 1)], o[j >> 1], 0, 0, 0);
    if (j < 4) f[j & 3] = FRAG(j + 28);
    else if (NEXT) f[j & 3] = N.k(0, j - 4);
    ANIMA_SB();
  }
#undef PROB2
#undef FRAG
}
#undef ANIMA_SB

// 4 waves x 32 queries per workgroup; K/V blocks of KB keys double-buffered in LDS, the next
// block prefetched into registers while the current one is consumed (one barrier per block).
template <int KB, bool NORM, bool ROPE, bool QP = false>
__global__ __launch_bounds__(256, KB == 32 ? 3 : 2) void attn_flash_bf16(FlashArgs a) {
  using T = Tiles<KB>;
  constexpr int UK = KB / 16;  // uint4 per thread for each of the K and V^T block copies
  static_assert(UK == 2 || UK == 4, "32 or 64 keys per block");
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * T::STAGE];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = id / a.n_qt, qt = id - bh * a.n_qt;
  const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group;
  const int qi = qt * BQ + wave * 32 + lq;
  const int Lk = a.kv_len[b];
  // causal (app/gpu/kernels.js:49, limit = min(cols, row + 1)): this lane's keys end at lim; the
  // workgroup's last block holds the key of its last query, and blocks before key qt * BQ (its
  // first query) need no mask
  const int lim = a.causal ? min(Lk, qi + 1) : Lk;
  const int nkb = a.causal ? min((Lk + KB - 1) / KB, (qt * BQ + BQ + KB - 1) / KB) : (Lk + KB - 1) / KB;
  const int nfull = a.causal ? min(Lk / KB, qt * BQ / KB) : Lk / KB;

  bf16x8 qf[8];
  if constexpr (QP) {
    const bf16x8 z8 = {};
    const uint16_t* src = a.qp + (((int64_t)b * a.Lq + (qi < a.Lq ? qi : 0)) * a.H + h) * HD + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) qf[ks] = qi < a.Lq ? *(const bf16x8*)(src + 16 * ks) : z8;
  } else {
    float x[64];
    load_q<NORM, ROPE>(a, b, h, qi, hf, x);
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int j = 0; j < 8; j++) qf[ks][j] = to_bf16(x[8 * ks + j] * a.c);
  }

  // global -> LDS copy assignment: K row t/(256/KB), KB bytes at (t%(256/KB))*KB;
  // V^T row t/2, KB bytes (KB/2 keys) at (t%2)*KB/2 keys
  constexpr int TPR = 256 / KB;
  const int kr = tid / TPR, kc = tid % TPR, vr = tid >> 1, vc = tid & 1;
  const uint4* kg = (const uint4*)((const bf16*)a.kb + (((int64_t)b * a.Hkv + hk) * a.Lkp + kr) * HD + kc * (KB / 2));
  const uint4* vg = (const uint4*)((const bf16*)a.vt + (((int64_t)b * a.Hkv + hk) * HD + vr) * a.Lkp + vc * (KB / 2));
  // prefetch registers (named, not an array: arrays indexed inside these copies were not
  // promoted to registers by the compiler and went through scratch memory)
  uint4 k0, k1, k2, k3, v0, v1, v2, v3;
#define GLOAD(blk)                                                                          \
  {                                                                                         \
    const uint4* ks_ = kg + (int64_t)(blk) * (KB * HD / 8);                                 \
    const uint4* vs_ = vg + (int64_t)(blk) * (KB / 8);                                      \
    k0 = ks_[0]; k1 = ks_[1]; v0 = vs_[0]; v1 = vs_[1];                                     \
    if constexpr (UK == 4) { k2 = ks_[2]; k3 = ks_[3]; v2 = vs_[2]; v3 = vs_[3]; }          \
  }
#define LSTORE(st)                                                                          \
  {                                                                                         \
    uint4* kd_ = (uint4*)(smem + (st) * T::STAGE + kr * T::KSP + kc * (KB / 2));            \
    uint4* vd_ = (uint4*)(smem + (st) * T::STAGE + T::KTILE + vr * T::VSP + vc * (KB / 2)); \
    kd_[0] = k0; kd_[1] = k1; vd_[0] = v0; vd_[1] = v1;                                     \
    if constexpr (UK == 4) { kd_[2] = k2; kd_[3] = k3; vd_[2] = v2; vd_[3] = v3; }          \
  }

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = (f32x16){};
  float m = 0.0f, l = 0.0f;
  f32x16 negm = {};

  GLOAD(0);
  LSTORE(0);
  __syncthreads();
  // Block 0 sets the offset.  Blocks from nfull on (the partial last block; with causal also
  // the blocks on the diagonal) take the key mask with this lane's limit.
  if (nkb > 1) GLOAD(1);
  if (nfull > 0) flash_block<KB, false, true>(PadAddr<KB>(smem, smem + T::KTILE, lq, hf), qf, o, m, negm, l, 0, Lk, hf);
  else flash_block<KB, true, true>(PadAddr<KB>(smem, smem + T::KTILE, lq, hf), qf, o, m, negm, l, 0, lim, hf);
  if (nkb > 1) LSTORE(1);
  __syncthreads();
  for (int kb = 1; kb < nfull; kb++) {
    const int st = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) GLOAD(kb + 1);
    if constexpr (KB == 64) {
      const PadAddr<KB> A(smem + st * T::STAGE, smem + st * T::STAGE + T::KTILE, lq, hf);
      bf16x8 f[4] = {A.k(0, 0), A.k(0, 1), A.k(0, 2), A.k(0, 3)};
      flash_block_main<PadAddr<KB>, false>(A, A, f, qf, o, m, negm, l);
    } else
      flash_block<KB, false, false>(PadAddr<KB>(smem + st * T::STAGE, smem + st * T::STAGE + T::KTILE, lq, hf), qf, o,
                                    m, negm, l, kb * KB, Lk, hf);
    if (more) LSTORE(st ^ 1);
    __syncthreads();
  }
  // masked blocks (a separate loop: in the main loop's body the masked block raised its registers
  // past the limit); block max(1, nfull) is already in its stage
  for (int kb = nfull > 1 ? nfull : 1; kb < nkb; kb++) {
    const int st = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) GLOAD(kb + 1);
    flash_block<KB, true, false>(PadAddr<KB>(smem + st * T::STAGE, smem + st * T::STAGE + T::KTILE, lq, hf), qf, o, m,
                                 negm, l, kb * KB, lim, hf);
    if (more) LSTORE(st ^ 1);
    __syncthreads();
  }
#undef GLOAD
#undef LSTORE

  l = pair_sum(l);
  if (qi < a.Lq) {
    const float inv = 1.0f / l;
    const int64_t off = (int64_t)b * a.o_bs + (int64_t)qi * a.ldo + h * a.D + 4 * hf;
    float* dst = a.o + off;
    bf16* dst16 = (bf16*)a.o + off;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
      if (32 * dt < a.D)  // D = 64: dim tiles 2, 3 are padding
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4 v =
              make_float4(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
          if (a.obf) *(bf16x4*)(dst16 + 32 * dt + 8 * g) = bf16x4{to_bf16(v.x), to_bf16(v.y), to_bf16(v.z), to_bf16(v.w)};
          else *(float4*)(dst + 32 * dt + 8 * g) = v;
        }
  }
}
constexpr int FLASH_KB = 64;  // keys per block of the bf16 kernel

// ------------------------------------------------------------------ bf16 kernel, 8 waves

// attn_flash_w8: one workgroup = 8 waves x 32 queries (two waves per SIMD, the per-wave block
// code of attn_flash_bf16), so each K/V block copied into LDS serves 256 queries (half the copy
// traffic per query of the 4-wave kernel).  Blocks of 64 keys go straight from global memory
// into four swizzled LDS stages (buffer_load ... lds, no register staging), issued three blocks
// ahead of the compute and published one block ahead, so that each block's first fragments are
// read while the previous block's last MFMAs run.
constexpr int W8_BQ = 256;
constexpr int W8_KB = 64;
constexpr int W8_ST = 2 * SWZ_KT;  // stage bytes: K tile + V^T tile
constexpr int W8_NST = 4;
constexpr int W8_OROW = 64 + 4;  // floats per row of the output staging (padded against bank conflicts)
static_assert(8 * 32 * W8_OROW * 4 <= W8_NST * W8_ST, "output staging must fit in the stages");

typedef __attribute__((address_space(3))) void lds_void_t;

// Lane byte offsets (relative to the block's first K row / first V^T key) of this wave's share
// of a block: 2 + 2 copies of one KiB (K rows 4i..4i+3 and V^T dim rows 8i..8i+7 for
// i = 2*wave + c), lanes permuted so that the LDS image is the swizzled layout.
struct W8Load {
  int k[2], v[2];
  __device__ __forceinline__ W8Load(int64_t lkp, int wave, int lane) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int i = 2 * wave + c;
      const int row = 4 * i + (lane >> 4);
      k[c] = row * (HD * 2) + 16 * ((lane & 15) ^ (row & 15));
      const int d = 8 * i + (lane >> 3);
      v[c] = (int)(d * lkp * 2) + 16 * ((lane & 7) ^ ((d >> 1) & 7));
    }
  }
};

// Buffer resources over one head's K rows and V^T rows (raw buffers, byte offsets; reads past
// num_records return zero).
struct W8Src {
  __amdgpu_buffer_rsrc_t k, v;
};

// Waves 0-3 (one per SIMD) issue all of a block's copies: their own chunks and those of wave
// w + 4 (K rows + 32 and V^T dims + 64, which keep the same lane permutation), so the other wave
// of each SIMD runs without copy and M0 set-up instructions.  vhalf: byte distance of 64 V^T rows.
__device__ __forceinline__ void w8_load(const W8Src& src, const W8Load& lo, int blk, char* stage, int wave, int vhalf) {
  if (wave >= 4) return;
#pragma unroll
  for (int h = 0; h < 2; h++) {
#pragma unroll
    for (int c = 0; c < 2; c++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.k, (lds_void_t*)(stage + (2 * wave + 8 * h + c) * 1024), 16, lo.k[c],
                                               blk * (W8_KB * HD * 2) + h * (32 * HD * 2), 0, 0);
#pragma unroll
    for (int c = 0; c < 2; c++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.v, (lds_void_t*)(stage + SWZ_KT + (2 * wave + 8 * h + c) * 1024), 16,
                                               lo.v[c], blk * (W8_KB * 2) + h * vhalf, 0, 0);
  }
}

// Workgroup barrier without a memory fence: the LDS copies a barrier publishes are covered by
// the explicit vmcnt waits before it, and LDS reads are complete once their MFMAs have issued.
// The empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void w8_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// vmcnt(n) only (expcnt and lgkmcnt at their no-wait maxima), gfx9 s_waitcnt encoding.
#define W8_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

// Q rows of one wave (32 queries x 128 fp32) reach the MFMA layout through LDS: per round of 64
// dims, eight lane-contiguous copies of 4 rows x 256 bytes each (whole lines per instruction;
// lane l -> row 4 i + l / 16, 16-byte slot l % 16 holding piece (slot ^ row) % 16 of the row), then
// each lane reads its row's pieces 4 ks + 2 hf, + 1.  Loaded straight into the MFMA layout, one
// instruction would touch 32 rows with one 16-byte access each, which the vector memory address
// path serves at about one access per clock.
constexpr int W8_QB = 8192;  // one wave's staging bytes: 32 rows x 64 fp32
__device__ __forceinline__ void w8_q_issue(__amdgpu_buffer_rsrc_t rq, char* qs, const int (&qo)[8], int round) {
#pragma unroll
  for (int i = 0; i < 8; i++)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void_t*)(qs + i * 1024), 16, qo[i] + 256 * round, 0, 0, 0);
}
// The prepared bf16 Q fragments (piece 2 ks + hf of the row for k-step ks) from the staging.
__device__ __forceinline__ void w8_qp_read(const char* __restrict__ qs, int lq, int hf, bf16x8 (&qf)[8]) {
#pragma unroll
  for (int ks = 0; ks < 8; ks++) qf[ks] = *(const bf16x8*)(qs + lq * 256 + 16 * ((2 * ks + hf) ^ (lq & 7)));
  asm volatile("" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]), "+v"(qf[4]), "+v"(qf[5]), "+v"(qf[6]), "+v"(qf[7]));
}
// (restrict: the reads carry alias scopes, so the compiler does not make them wait for the K / V
// copies in flight; whole 16-byte vectors, which keep them)
__device__ __forceinline__ void w8_q_read(const char* __restrict__ qs, int lq, int hf, float* x) {
  f32x4 v[8];
#pragma unroll
  for (int p = 0; p < 8; p++) v[p] = *(const f32x4*)(qs + lq * 256 + 16 * ((4 * (p >> 1) + 2 * hf + (p & 1)) ^ (lq & 7)));
  asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
#pragma unroll
  for (int p = 0; p < 8; p++)
#pragma unroll
    for (int e = 0; e < 4; e++) x[4 * p + e] = v[p][e];
}

template <bool NORM, bool ROPE, bool QP = false>
__global__ __launch_bounds__(512, 1) void attn_flash_w8(FlashArgs a) {
  // the K / V stages, then 32 KiB that with stage 3 stage Q in the prologue
  __shared__ __attribute__((aligned(1024))) char smem[W8_NST * W8_ST + 32768];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = id / a.n_qt, qt = id - bh * a.n_qt;
  const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group;
  const int qi = qt * W8_BQ + wave * 32 + lq;
  const int Lk = a.kv_len[b];
  const int nkb = (Lk + W8_KB - 1) / W8_KB;
  const int head_bytes = a.Lkp * HD * 2;
  W8Src src;
  src.k = __builtin_amdgcn_make_buffer_rsrc((void*)((const bf16*)a.kb + ((int64_t)b * a.Hkv + hk) * a.Lkp * HD), (short)0,
                                            head_bytes, 0x00020000);
  src.v = __builtin_amdgcn_make_buffer_rsrc((void*)((const bf16*)a.vt + ((int64_t)b * a.Hkv + hk) * HD * a.Lkp), (short)0,
                                            head_bytes, 0x00020000);

  // Q's first 64 dims are copied first, then K / V blocks 0, 1 and 2, so the wait for Q leaves
  // those in flight (rows past Lq read zeros)
  const int qrow0 = qt * W8_BQ, nrow = a.Lq - qrow0 < W8_BQ ? a.Lq - qrow0 : W8_BQ;
  char* qs = smem + 3 * W8_ST + wave * W8_QB;
  int qo[8];
  __amdgpu_buffer_rsrc_t rq;
  if constexpr (QP) {
    // prepared Q: one copy round of the wave's 32 rows x 256 bytes (16-byte pieces swizzled as
    // for fp32 Q, 16 per row)
    rq = __builtin_amdgcn_make_buffer_rsrc((void*)(a.qp + (((int64_t)b * a.Lq + qrow0) * a.H + h) * HD), (short)0,
                                           nrow * a.H * HD * 2, 0x00020000);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int row = 4 * i + (lane >> 4);
      qo[i] = (wave * 32 + row) * a.H * HD * 2 + 16 * ((lane & 15) ^ (row & 7));
    }
  } else {
    rq = __builtin_amdgcn_make_buffer_rsrc((void*)(a.q + (int64_t)b * a.q_bs + (int64_t)qrow0 * a.ldq + h * a.D),
                                           (short)0, nrow * (int)a.ldq * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int row = 4 * i + (lane >> 4);
      qo[i] = ((wave * 32 + row) * (int)a.ldq + 4 * ((lane & 15) ^ (row & 7))) * 4;
    }
  }
  w8_q_issue(rq, qs, qo, 0);
  const W8Load lo(a.Lkp, wave, lane);
  const int vhalf = 64 * a.Lkp * 2;
  w8_load(src, lo, 0, smem, wave, vhalf);
  if (nkb > 1) w8_load(src, lo, 1, smem + W8_ST, wave, vhalf);
  if (nkb > 2) w8_load(src, lo, 2, smem + 2 * W8_ST, wave, vhalf);

  bf16x8 qf[8];
  // waves 0-3 issued 8 K / V copies per block after Q's
  if (wave >= 4) W8_WAIT_VM(0);
  else if (nkb > 2) W8_WAIT_VM(24);
  else if (nkb > 1) W8_WAIT_VM(16);
  else W8_WAIT_VM(8);
  if constexpr (QP) {
    w8_qp_read(qs, lq, hf, qf);
  } else {
    float x[64];
    w8_q_read(qs, lq, hf, x);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the reads are done before the refill
    w8_q_issue(rq, qs, qo, 1);
    W8_WAIT_VM(0);
    w8_q_read(qs, lq, hf, x + 32);
    q_norm<NORM>(a, hf, x);
    if constexpr (ROPE) {
      // the rows' cos and sin (64 fp32 each) through the same staging, rows past Lq reading zeros
      // (their Q is zero)
      const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(a.cs + (int64_t)qrow0 * (HD / 2)), (short)0, nrow * (HD / 2) * 4, 0x00020000);
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(a.cs + a.sin_off + (int64_t)qrow0 * (HD / 2)), (short)0, nrow * (HD / 2) * 4, 0x00020000);
      int co[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int row = 4 * i + (lane >> 4);
        co[i] = ((wave * 32 + row) * (HD / 2) + 4 * ((lane & 15) ^ (row & 7))) * 4;
      }
      float c[32], sn[32];
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      w8_q_issue(rc, qs, co, 0);
      W8_WAIT_VM(0);
      w8_q_read(qs, lq, hf, c);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      w8_q_issue(rs, qs, co, 0);
      W8_WAIT_VM(0);
      w8_q_read(qs, lq, hf, sn);
      q_rope(x, c, sn);
    }
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int j = 0; j < 8; j++) qf[ks][j] = to_bf16(x[8 * ks + j] * a.c);
  }
  const SwzOfs of(lq, hf);
  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = (f32x16){};
  float m = 0.0f, l = 0.0f;
  f32x16 negm = {};

  // Block j lives in stage j % 4.  The barrier at the top of iteration j publishes block j+1 (a
  // wave first waits for its own copies of it; the 8 of block j+2 may still be in flight), so
  // block j's last MFMAs can carry the reads of block j+1's first fragments.  The barrier also
  // ends every wave's reads of block j-1, whose stage is then refilled with block j+3.  The
  // barrier before block 0 publishes blocks 0 and 1; a partial last block needs no barrier of
  // its own (published one iteration ahead, and its stage is not refilled).
  const int nfull = Lk / W8_KB;
  if (nkb > 2) W8_WAIT_VM(8);
  else W8_WAIT_VM(0);
  w8_barrier();
  if (nkb > 3) w8_load(src, lo, 3, smem + 3 * W8_ST, wave, vhalf);
  if (nfull > 0) flash_block<W8_KB, false, true>(SwzAddr(smem, of), qf, o, m, negm, l, 0, Lk, hf);
  else flash_block<W8_KB, true, true>(SwzAddr(smem, of), qf, o, m, negm, l, 0, Lk, hf);
  bf16x8 f[4];
  {
    const SwzAddr A1(smem + W8_ST, of);
#pragma unroll
    for (int i = 0; i < 4; i++) f[i] = A1.k(0, i);
  }
  // The loop is unrolled over the four stages so that every LDS address is a lane offset plus an
  // immediate: stages 0 and 1 use the offsets of `of`, stages 2 and 3 those of `of2` (+64 KiB),
  // which keeps each immediate below 64 KiB.
  const SwzOfs of2(lq, hf, 2 * W8_ST);
#define W8_ADDR(ST) SwzAddr(smem + ((ST) & 1) * W8_ST, (ST) < 2 ? of : of2)
#define W8_ITER(ST)                                                                                    \
  {                                                                                                    \
    if (j >= nfull) break;                                                                             \
    if (j + 2 < nkb) W8_WAIT_VM(8);                                                                    \
    else W8_WAIT_VM(0);                                                                                \
    w8_barrier();                                                                                      \
    if (j + 3 < nkb) w8_load(src, lo, j + 3, smem + (((ST) + 3) & 3) * W8_ST, wave, vhalf);            \
    flash_block_main<SwzAddr, true>(W8_ADDR(ST), W8_ADDR(((ST) + 1) & 3), f, qf, o, m, negm, l);        \
    j++;                                                                                               \
  }
  for (int j = 1;;) {
    W8_ITER(1)
    W8_ITER(2)
    W8_ITER(3)
    W8_ITER(0)
  }
#undef W8_ITER
#undef W8_ADDR
  if (nfull < nkb && nfull > 0)
    flash_block<W8_KB, true, false>(SwzAddr(smem + (nfull & 3) * W8_ST, of), qf, o, m, negm, l, nfull * W8_KB, Lk, hf);

  l = pair_sum(l);
  const float inv = 1.0f / l;
  // The output leaves through LDS so that every store instruction writes whole 256-byte row
  // segments: straight from the MFMA layout each instruction would put 32 bytes into each of 32
  // rows, and the partially written lines double the HBM write traffic.  Each wave transposes its
  // own 32 x 128 block in two 64-column halves through a private slice of the (now idle) stages.
  w8_barrier();  // every wave is done reading the key/value stages
  float* ow = (float*)smem + wave * (32 * W8_OROW);
  const int rr = lane >> 4, cc = 4 * (lane & 15);
  float* dst = a.o + (int64_t)b * a.o_bs + h * HD + cc;
  bf16* dst16 = (bf16*)a.o + (int64_t)b * a.o_bs + h * HD + cc;
  const int q0 = qt * W8_BQ + wave * 32;
#pragma unroll
  for (int half = 0; half < 2; half++) {
#pragma unroll
    for (int d2 = 0; d2 < 2; d2++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const f32x16& v = o[2 * half + d2];
        *(float4*)(ow + lq * W8_OROW + 32 * d2 + 8 * g + 4 * hf) =
            make_float4(v[4 * g] * inv, v[4 * g + 1] * inv, v[4 * g + 2] * inv, v[4 * g + 3] * inv);
      }
    // one wave's LDS accesses complete in program order: no wait between these writes and reads
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int r = 4 * k + rr;
      const float4 v = *(const float4*)(ow + r * W8_OROW + cc);
      if (q0 + r < a.Lq) {
        if (a.obf)
          *(bf16x4*)(dst16 + (int64_t)(q0 + r) * a.ldo + 64 * half) =
              bf16x4{to_bf16(v.x), to_bf16(v.y), to_bf16(v.z), to_bf16(v.w)};
        else
          *(float4*)(dst + (int64_t)(q0 + r) * a.ldo + 64 * half) = v;
      }
    }
  }
}
#undef W8_WAIT_VM

// ------------------------------------------------------------------ fp32 MFMA kernel

constexpr int KSP32 = HD + 4;  // floats
constexpr int VSP32 = BK + 4;

template <bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void attn_flash_fp32(FlashArgs a) {
  __shared__ __attribute__((aligned(16))) float Ks[BK * KSP32];
  __shared__ __attribute__((aligned(16))) float Vs[HD * VSP32];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, hf = lane >> 5;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = id / a.n_qt, qt = id - bh * a.n_qt;
  const int b = bh / a.H, h = bh - b * a.H, hk = h / a.group;
  const int qi = qt * BQ + wave * 32 + lq;
  const int Lk = a.kv_len[b];
  // causal: as in attn_flash_bf16 (lim: this lane's key limit; mlim: the workgroup's smallest)
  const int lim = a.causal ? min(Lk, qi + 1) : Lk;
  const int mlim = a.causal ? min(Lk, qt * BQ + 1) : Lk;
  const int nkb = a.causal ? min((Lk + BK - 1) / BK, (qt * BQ + BQ + BK - 1) / BK) : (Lk + BK - 1) / BK;

  // lane keeps Q[qi][2ks + hf] for ks = 0..63 (K-group g of a 32x32x2 MFMA = dim parity)
  float qv[64];
  {
    float x[64];
    load_q<NORM, ROPE>(a, b, h, qi, hf, x);
    // x holds dims 16ks8 + 8hf + j; redistribute across the lane pair so that lane (q, g)
    // holds the dims of parity g.  Lane hf has dims {16k + 8hf + j}; exchange with lane^32.
#pragma unroll
    for (int k8 = 0; k8 < 8; k8++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float mine = x[8 * k8 + j];
        const float other = __shfl_xor(mine, 32);
        // dim of `mine` = 16k8 + 8hf + j, of `other` = 16k8 + 8(1-hf) + j
        const float lo = hf ? other : mine;  // dim 16k8 + j
        const float hi = hf ? mine : other;   // dim 16k8 + 8 + j
        // keep dims with parity hf: d = 2ks + hf
        if ((j & 1) == hf) {
          qv[(16 * k8 + j) >> 1] = lo;
          qv[(16 * k8 + 8 + j) >> 1] = hi;
        }
      }
  }

  const float* kg = (const float*)a.kb + ((int64_t)b * a.Hkv + hk) * a.Lkp * HD;
  const float* vg = (const float*)a.vt + ((int64_t)b * a.Hkv + hk) * HD * a.Lkp;
  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = (f32x16){};
  float m = -INFINITY, l = 0.0f;

  for (int kb = 0; kb < nkb; kb++) {
    // K tile 64 x 128 floats: thread -> row t/4, 32 floats; V^T tile 128 x 64: row t/2, 32 floats
    {
      const float4* ks = (const float4*)(kg + ((int64_t)kb * BK + (tid >> 2)) * HD + 32 * (tid & 3));
      float4* kd = (float4*)(Ks + (tid >> 2) * KSP32 + 32 * (tid & 3));
      const float4* vsrc = (const float4*)(vg + (int64_t)(tid >> 1) * a.Lkp + kb * BK + 32 * (tid & 1));
      float4* vd = (float4*)(Vs + (tid >> 1) * VSP32 + 32 * (tid & 1));
#pragma unroll
      for (int i = 0; i < 8; i++) {
        kd[i] = ks[i];
        vd[i] = vsrc[i];
      }
    }
    __syncthreads();
    f32x16 s0 = {}, s1 = {};
#pragma unroll 16
    for (int ks = 0; ks < 64; ks++) {
      const float k0 = Ks[lq * KSP32 + 2 * ks + hf];
      const float k1 = Ks[(32 + lq) * KSP32 + 2 * ks + hf];
      s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(k0, qv[ks], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(k1, qv[ks], s1, 0, 0, 0);
    }
    if ((kb + 1) * BK > mlim) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int key = kb * BK + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (key >= lim) s0[r] = -INFINITY;
        if (key + 32 >= lim) s1[r] = -INFINITY;
      }
    }
    float bm = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int r = 1; r < 16; r++) bm = fmaxf(bm, fmaxf(s0[r], s1[r]));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float bmc = bm * a.c;
    const bool need = bmc > m + RESCALE_SLACK;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = need ? ceilf(bmc) : m;
      const float alpha = __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] *= alpha;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      s0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], a.c, -m));
      s1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], a.c, -m));
      l += s0[r] + s1[r];
    }
    // k-step (tile t, register r): keys 32t + 8(r/4) + 4g + r%4 for k-group g
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
#pragma unroll
      for (int dt = 0; dt < 4; dt++) {
        const float* vrow = Vs + (32 * dt + lq) * VSP32;
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[key], s0[r], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 + key], s1[r], o[dt], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  l += __shfl_xor(l, 32);
  if (qi < a.Lq) {
    const float inv = 1.0f / l;
    float* dst = a.o + (int64_t)b * a.o_bs + (int64_t)qi * a.ldo + h * a.D + 4 * hf;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
      if (32 * dt < a.D)  // D = 64: dim tiles 2, 3 are padding
#pragma unroll
        for (int g = 0; g < 4; g++)
          *(float4*)(dst + 32 * dt + 8 * g) =
              make_float4(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
  }
}

// ------------------------------------------------------------------ host launcher

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Argument checks of anima_attention (fills kv_len[] with the valid key counts).
static int attention_check(anima_ctx* c, const anima_attn_desc* d, int (&kv_len)[MAXB]) {
  const int group = d->group <= 0 ? 1 : d->group;
  if (d->D != HD && d->D != HD / 2)
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention: head dim %d on the flash kernels (D = 128 or 64)", d->D);
  if (d->D != HD && (d->q_norm || d->k_norm || d->rope_cs || d->kv_prep))
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention: fused q/k norm, RoPE and prepared K/V need D = 128 (D = %d)", d->D);
  if (d->B < 1 || d->B > MAXB) return fail(c, ANIMA_E_ARG, "anima_attention: B=%d outside [1,%d]", d->B, MAXB);
  if (d->Lq < 1 || d->Lk < 1 || d->H < 1) return fail(c, ANIMA_E_ARG, "anima_attention: Lq=%d Lk=%d H=%d must be >= 1", d->Lq, d->Lk, d->H);
  if (d->Lk > (1 << 22)) return fail(c, ANIMA_E_ARG, "anima_attention: Lk=%d (at most %d keys)", d->Lk, 1 << 22);
  if (d->H % group) return fail(c, ANIMA_E_ARG, "anima_attention: H=%d not a multiple of group=%d", d->H, group);
  const bool prepared = d->kv_prep != nullptr, qprep = d->q_prep != nullptr;
  if ((!d->q && !qprep) || !d->o || (!prepared && (!d->k || !d->v))) return fail(c, ANIMA_E_ARG, "anima_attention: null q/k/v/o");
  if (qprep && (d->precision != ANIMA_PREC_BF16 || d->D != HD || !al16(d->q_prep)))
    return fail(c, ANIMA_E_ARG, "anima_attention: a prepared Q needs bf16 precision, D = 128 and 16-byte alignment");
  if (d->precision != ANIMA_PREC_BF16 && d->precision != ANIMA_PREC_FP32)
    return fail(c, ANIMA_E_ARG, "anima_attention: unknown precision %d", d->precision);
  if (d->o_bf16 && d->precision != ANIMA_PREC_BF16)
    return fail(c, ANIMA_E_ARG, "anima_attention: a bf16 O needs bf16 precision");
  const int64_t lds[4] = {d->ldq, d->ldk, d->ldv, d->ldo};
  const int64_t offs[4] = {d->q_off, d->k_off, d->v_off, d->o_off};
  const int64_t bss[4] = {d->q_bstride, d->k_bstride, d->v_bstride, d->o_bstride};
  const char* nm[4] = {"q", "k", "v", "o"};
  const int heads[4] = {d->H, d->H / group, d->H / group, d->H};
  for (int i = 0; i < 4; i++) {
    if (prepared && (i == 1 || i == 2)) continue;  // K / V come converted
    if (qprep && i == 0) continue;                 // Q comes prepared
    if (lds[i] % 4 || offs[i] % 4 || bss[i] % 4 || lds[i] < 0 || offs[i] < 0 || bss[i] < 0)
      return fail(c, ANIMA_E_ARG, "anima_attention: %s ld/off/bstride (%lld/%lld/%lld) must be non-negative multiples of 4 (vec4 rows, as ops.js:169)",
                  nm[i], (long long)lds[i], (long long)offs[i], (long long)bss[i]);
    if (lds[i] < offs[i] + (int64_t)heads[i] * d->D)
      return fail(c, ANIMA_E_ARG, "anima_attention: %s rows of %lld elements cannot hold off %lld + %d heads x %d", nm[i],
                  (long long)lds[i], (long long)offs[i], heads[i], d->D);
  }
  if ((!qprep && !al16(d->q)) || !al16(d->o) || (!prepared && (!al16(d->k) || !al16(d->v))) || (prepared && !al16(d->kv_prep)))
    return fail(c, ANIMA_E_ARG, "anima_attention: q/k/v/o (or kv_prep) must be 16-byte aligned");
  if ((d->q_norm && !al16(d->q_norm)) || (d->k_norm && !al16(d->k_norm)))
    return fail(c, ANIMA_E_ARG, "anima_attention: q_norm/k_norm must be 16-byte aligned");
  for (int b = 0; b < d->B; b++) {
    kv_len[b] = d->kv_len ? d->kv_len[b] : d->Lk;
    if (kv_len[b] < 1 || kv_len[b] > d->Lk) return fail(c, ANIMA_E_ARG, "anima_attention: kv_len[%d]=%d outside [1, Lk=%d]", b, kv_len[b], d->Lk);
  }
  if (prepared && d->kv_prep_bytes != attention_kv_bytes(d->B, d->H / group, d->Lk, d->precision))
    return fail(c, ANIMA_E_ARG, "anima_attention: kv_prep_bytes=%lld, but B=%d, %d kv heads, Lk=%d at this precision take %lld",
                (long long)d->kv_prep_bytes, d->B, d->H / group, d->Lk,
                (long long)attention_kv_bytes(d->B, d->H / group, d->Lk, d->precision));
  const bool rope = d->rope_cs != nullptr;
  if (rope) {
    const int64_t rows = d->rope_sin_off / (HD / 2);
    if (d->rope_sin_off <= 0 || d->rope_sin_off % (HD / 2) || rows < d->Lq || rows < d->Lk)
      return fail(c, ANIMA_E_ARG, "anima_attention: rope_sin_off=%lld must be rows*%d with rows >= max(Lq,Lk)=%d",
                  (long long)d->rope_sin_off, HD / 2, d->Lq > d->Lk ? d->Lq : d->Lk);
    if (!al16(d->rope_cs)) return fail(c, ANIMA_E_ARG, "anima_attention: rope_cs must be 16-byte aligned");
  }
  return ANIMA_OK;
}

// The K/V prep of one attention call into dst ([K plane][V^T plane], each B Hkv Lkp HD elements).
static int prep_kv_launch(anima_ctx* c, const anima_attn_desc* d, void* dst) {
  const int group = d->group <= 0 ? 1 : d->group;
  const int Hkv = d->H / group;
  const int Lkp = (d->Lk + BK - 1) / BK * BK;
  const bool bf = d->precision == ANIMA_PREC_BF16;
  const bool rope = d->rope_cs != nullptr;
  const float eps = d->eps;
  const size_t plane = (size_t)d->B * Hkv * Lkp * HD * (bf ? 2 : 4);
  int rc = ANIMA_OK;
  PrepArgs p;
  p.k = d->k + d->k_off;
  p.ldk = d->ldk;
  p.k_bs = d->k_bstride;
  p.v = d->v + d->v_off;
  p.ldv = d->ldv;
  p.v_bs = d->v_bstride;
  p.kb = dst;
  p.vt = (char*)dst + plane;
  p.kn = d->k_norm;
  p.cs = d->rope_cs;
  p.sin_off = d->rope_sin_off;
  p.eps = eps;
  p.Hkv = Hkv;
  p.Lk = d->Lk;
  p.Lkp = Lkp;
  p.D = d->D;
  {
    const double bytes = (double)d->B * Hkv * d->Lk * d->D * 4 * 2 + 2.0 * plane;
    Launch L(c, bf ? "attn.prep_kv_bf16" : "attn.prep_kv_fp32", 0.0, bytes);
    dim3 grid(Hkv, Lkp / BK, d->B);  // heads fastest: concurrent workgroups read whole K / V rows
    const dim3 grid_lines(Lkp / BK, Hkv, d->B);  // key blocks fastest (attn_prep_kv_lines)
    const bool kn = d->k_norm != nullptr;
#define PREP(T, N, R) hipLaunchKernelGGL((attn_prep_kv<T, N, R>), grid, dim3(256), 0, c->stream, p)
#define PREP_LINES(N, R) hipLaunchKernelGGL((attn_prep_kv_lines<N, R>), grid_lines, dim3(256), 0, c->stream, p)
    if (bf) {
      if (kn && rope) PREP_LINES(true, true);
      else if (kn) PREP_LINES(true, false);
      else if (rope) PREP_LINES(false, true);
      else PREP_LINES(false, false);
    } else {
      if (kn && rope) PREP(float, true, true);
      else if (kn) PREP(float, true, false);
      else if (rope) PREP(float, false, true);
      else PREP(float, false, false);
    }
#undef PREP
#undef PREP_LINES
    if ((rc = L.end())) return rc;
  }

  return ANIMA_OK;
}

int attention_launch(anima_ctx* c, const anima_attn_desc* d) { return attention_launch_ws(c, d, nullptr); }

// scratch != nullptr: the K/V prep goes there (the caller checked its size) instead of the
// context's workspace.
int attention_launch_ws(anima_ctx* c, const anima_attn_desc* d, void* scratch) {
  if (scratch && d->D != HD) return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention_noalloc: head dim %d", d->D);
  // D = 64 without fused norm / RoPE / prepared K/V (the LLM adapter's heads, dit.js:147-160):
  // the flash kernels with the operands zero-padded to 128 dims (flashAttentionShader(64) of
  // ops.js:170); any other head dim: the chunked path (app/gpu/ops.js:177-207)
  const bool flash64 = d->D == HD / 2 && !d->q_norm && !d->k_norm && !d->rope_cs && !d->kv_prep;
  if (d->D != HD && !flash64) {
    if (d->o_bf16) return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention: a bf16 O on the chunked path (head dim %d)", d->D);
    int rc = attention_chunked_check(c, d);
    if (rc) return rc;
    int kvl[MAXB];
    if (d->B > MAXB) return fail(c, ANIMA_E_ARG, "anima_attention: B=%d above %d", d->B, MAXB);
    for (int b = 0; b < d->B; b++) {
      kvl[b] = d->kv_len ? d->kv_len[b] : d->Lk;
      if (kvl[b] < 1 || kvl[b] > d->Lk) return fail(c, ANIMA_E_ARG, "anima_attention: kv_len[%d]=%d outside [1, Lk=%d]", b, kvl[b], d->Lk);
    }
    return attention_chunked_launch(c, d, kvl);
  }
  int kv_len[MAXB];
  int rc = attention_check(c, d, kv_len);
  if (rc) return rc;
  const int group = d->group <= 0 ? 1 : d->group;
  const bool rope = d->rope_cs != nullptr;
  const float scale = d->scale != 0.0f ? d->scale : 1.0f / sqrtf((float)d->D);
  const float eps = d->eps;
  const int Hkv = d->H / group;
  const int Lkp = (d->Lk + BK - 1) / BK * BK;
  const bool bf = d->precision == ANIMA_PREC_BF16;
  const size_t esz = bf ? 2 : 4;
  const size_t plane = (size_t)d->B * Hkv * Lkp * HD * esz;
  void* ws = (void*)d->kv_prep;
  if (!ws) {
    if (scratch) ws = scratch;
    else if ((rc = workspace(c, 2 * plane, &ws))) return rc;
    if ((rc = prep_kv_launch(c, d, ws))) return rc;
  }

  FlashArgs f;
  f.q = d->q ? d->q + d->q_off : nullptr;
  f.ldq = d->ldq;
  f.q_bs = d->q_bstride;
  f.kb = ws;
  f.vt = (char*)ws + plane;
  // (with a bf16 O the offset counts uint16 elements)
  f.o = d->o_bf16 ? (float*)((uint16_t*)d->o + d->o_off) : d->o + d->o_off;
  f.ldo = d->ldo;
  f.o_bs = d->o_bstride;
  f.qn = d->q_norm;
  f.cs = d->rope_cs;
  f.sin_off = d->rope_sin_off;
  f.eps = eps;
  f.c = scale * 1.4426950408889634f;
  f.H = d->H;
  f.group = group;
  f.Hkv = Hkv;
  f.Lq = d->Lq;
  f.Lkp = Lkp;
  // 8-wave workgroups (256 queries) when that grid still gives every CU a workgroup
  // (the Q copies of a workgroup use 32-bit offsets: 256 rows of ldq fp32)
  const bool w8 = bf && !d->causal && d->D == HD && (int64_t)((d->Lq + W8_BQ - 1) / W8_BQ) * d->H * d->B >= c->num_cus &&
                  (int64_t)W8_BQ * (d->q_prep ? d->H * HD / 2 : d->ldq) * 4 < (1LL << 31);
  f.n_qt = w8 ? (d->Lq + W8_BQ - 1) / W8_BQ : (d->Lq + BQ - 1) / BQ;
  for (int b = 0; b < MAXB; b++) f.kv_len[b] = b < d->B ? kv_len[b] : 1;
  f.causal = d->causal ? 1 : 0;
  f.D = d->D;
  f.qp = (const uint16_t*)d->q_prep;
  f.obf = d->o_bf16 ? 1 : 0;
  double flops = 0;
  for (int b = 0; b < d->B; b++) flops += 4.0 * d->Lq * (double)kv_len[b] * d->D * d->H;
  const int blocks = f.n_qt * d->H * d->B;
  Launch L(c, w8 ? "attn.flash_bf16" : bf ? "attn.flash_bf16_4w" : "attn.flash_fp32", flops, 0.0);
  const bool qn = d->q_norm != nullptr;
#define FLASH(K, N, R) hipLaunchKernelGGL((K<N, R>), dim3(blocks), dim3(256), 0, c->stream, f)
#define FLASHB(T, N, R) hipLaunchKernelGGL((attn_flash_bf16<T, N, R>), dim3(blocks), dim3(256), 0, c->stream, f)
  if (f.qp && w8) {
    hipLaunchKernelGGL((attn_flash_w8<false, false, true>), dim3(blocks), dim3(512), 0, c->stream, f);
  } else if (f.qp) {
    hipLaunchKernelGGL((attn_flash_bf16<FLASH_KB, false, false, true>), dim3(blocks), dim3(256), 0, c->stream, f);
  } else if (w8) {
#define FLASH8(N, R) hipLaunchKernelGGL((attn_flash_w8<N, R>), dim3(blocks), dim3(512), 0, c->stream, f)
    if (qn && rope) FLASH8(true, true);
    else if (qn) FLASH8(true, false);
    else if (rope) FLASH8(false, true);
    else FLASH8(false, false);
#undef FLASH8
  } else if (bf) {
    if (qn && rope) FLASHB(FLASH_KB, true, true);
    else if (qn) FLASHB(FLASH_KB, true, false);
    else if (rope) FLASHB(FLASH_KB, false, true);
    else FLASHB(FLASH_KB, false, false);
  } else {
    if (qn && rope) FLASH(attn_flash_fp32, true, true);
    else if (qn) FLASH(attn_flash_fp32, true, false);
    else if (rope) FLASH(attn_flash_fp32, false, true);
    else FLASH(attn_flash_fp32, false, false);
  }
#undef FLASH
#undef FLASHB
  return L.end();
}

}  // namespace anima

namespace anima {

// ---- the no-allocation entry point's scratch: the K/V prep of anima_attention_noalloc lives in
// this file-scope device array (one per GPU, loaded with the code object, held until the process
// ends).  Host code never passes `scratch` itself to a kernel (in host code the name is a host-side
// stand-in): its device address is looked up once per device at context creation and kept.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static void* g_scratch_ptr[MAX_DEVICES];
static std::mutex g_scratch_mu;

int attention_scratch_init(anima_ctx* c) {
  if (c->device < 0 || c->device >= MAX_DEVICES)
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_init: device %d beyond the %d devices with a scratch address slot", c->device,
                MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[c->device]) {  // the caller made c->device current
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(c, e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[c->device] = ptr;
  }
  c->scratch = g_scratch_ptr[c->device];
  return ANIMA_OK;
}

size_t attention_scratch_bytes() { return NOALLOC_SCRATCH_BYTES; }

int attention_noalloc_launch(anima_ctx* c, const anima_attn_desc* d) {
  if (!d) return fail(c, ANIMA_E_ARG, "anima_attention_noalloc: null descriptor");
  if (d->D != HD)
    return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention_noalloc: head dim %d (the allocation-free path covers D=%d)", d->D, HD);
  if (!c->scratch) return fail(c, ANIMA_E_STATE, "anima_attention_noalloc: no scratch address for device %d", c->device);
  if (!d->kv_prep) {
    const int group = d->group <= 0 ? 1 : d->group;
    const int64_t need = (d->B >= 1 && d->H >= 1 && d->H % group == 0) ? attention_kv_bytes(d->B, d->H / group, d->Lk, d->precision) : 0;
    if (need > (int64_t)NOALLOC_SCRATCH_BYTES)
      return fail(c, ANIMA_E_ARG,
                  "anima_attention_noalloc: B=%d, %d kv heads, Lk=%d at this precision need %lld bytes of K/V scratch; the maximum is %zu",
                  d->B, d->H / group, d->Lk, (long long)need, NOALLOC_SCRATCH_BYTES);
  }
  // the profiler's event brackets may create events: none are taken during this call
  const bool prof = c->profiling;
  c->profiling = false;
  const int rc = attention_launch_ws(c, d, c->scratch);
  c->profiling = prof;
  return rc;
}

int64_t attention_kv_bytes(int B, int Hkv, int Lk, int precision) {
  if (B < 1 || Hkv < 1 || Lk < 1) return 0;
  const int64_t Lkp = (Lk + BK - 1) / BK * BK;
  return 2 * (int64_t)B * Hkv * Lkp * HD * (precision == ANIMA_PREC_BF16 ? 2 : 4);
}

int attention_prepare_kv_launch(anima_ctx* c, const anima_attn_desc* d, void* dst) {
  if (!d || !dst) return fail(c, ANIMA_E_ARG, "anima_attention_prepare_kv: null descriptor or output");
  if (d->kv_prep) return fail(c, ANIMA_E_ARG, "anima_attention_prepare_kv: desc->kv_prep must be NULL");
  if (!al16(dst)) return fail(c, ANIMA_E_ARG, "anima_attention_prepare_kv: kv_prep must be 16-byte aligned");
  const int group = d->group <= 0 ? 1 : d->group;
  if (d->D != HD) return fail(c, ANIMA_E_UNSUPPORTED, "anima_attention_prepare_kv: head dim %d (prepared K/V need D = 128)", d->D);
  if (d->kv_prep_bytes != attention_kv_bytes(d->B, d->H / group, d->Lk, d->precision))
    return fail(c, ANIMA_E_ARG, "anima_attention_prepare_kv: kv_prep_bytes=%lld, the layout takes %lld",
                (long long)d->kv_prep_bytes, (long long)attention_kv_bytes(d->B, d->H / group, d->Lk, d->precision));
  int kv_len[MAXB];
  int rc = attention_check(c, d, kv_len);  // the full call's checks (q / o included)
  if (rc) return rc;
  return prep_kv_launch(c, d, dst);
}
}  // namespace anima
