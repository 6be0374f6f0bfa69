// Device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace anima {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ bf16 to_bf16(float x) { return (bf16)x; }

// GELU with the Abramowitz-Stegun erf of app/gpu/kernels.js:11-18.  The reciprocal is v_rcp_f32
// (1 ulp) and the exponential v_exp_f32 (2^x) of -a^2 scaled by log2(e) (about 1 ulp plus the
// rounding of the scaled argument); the polynomial runs on FMAs, which WGSL lets the reference's
// compiler use as well.  Inside the accuracy WGSL grants the reference's division (2.5 ulp) and
// exp (3 + 2|x| ulp); against the correctly rounded formula the output differs by about 2e-8
// relative L2 on N(0, 9) inputs.  sign(z) * y is copysign(y, z): at z = 0 the result is 0.5 x
// either way (x = 0 there, or so small that y ~ 1e-9 vanishes in 1 + y).
__device__ __forceinline__ float gelu_erf(float x) {
  const float z = x * 0.7071067811865476f;
  const float a = fabsf(z);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, a, 1.0f));
  float p = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  p = __builtin_fmaf(p, t, 1.421413741f);
  p = __builtin_fmaf(p, t, -0.284496736f);
  p = __builtin_fmaf(p, t, 0.254829592f);
  const float e = __builtin_amdgcn_exp2f(a * a * -1.4426950408889634f);
  const float y = __builtin_fmaf(-(p * t), e, 1.0f);
  const float h = 0.5f * x;
  return __builtin_fmaf(h, __builtin_copysignf(y, z), h);
}

// The activations of the linear epilogues (ANIMA_ACT_*), shared by the GEMM epilogues and the
// row kernels that apply a linear's activation after the fact (anima_quant_rows_act).
__device__ __forceinline__ float silu_f(float r) { return r / (1.0f + expf(-r)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) v = fmaxf(v, __shfl_xor(v, s));
  return v;
}

// Pairwise tree over a wave in the order of a shared-memory "red[i] += red[i + s]" loop
// with s = n/2 ... 1 (lane 0 ends with the total).  n <= 64.
__device__ __forceinline__ float tree_sum_down(float v, int n) {
  for (int s = n / 2; s > 0; s >>= 1) v += __shfl_down(v, s);
  return v;
}

// Workgroup id -> work item.  Consecutive workgroup ids are dispatched round-robin over the 8
// XCDs; remapping gives each XCD a contiguous range of work items, so neighbouring items (one
// attention head's query tiles, one GEMM row of tiles) run on the same XCD and share its L2.
__device__ __forceinline__ int xcd_remap(int id, int total) {
  if ((total & 7) != 0) return id;
  return (id & 7) * (total >> 3) + (id >> 3);
}

}  // namespace anima
