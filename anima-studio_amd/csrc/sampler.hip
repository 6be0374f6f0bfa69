// One sampler step on the device (app/pipeline.js:276-283 CFG combine + denoised,
// app/samplers.js:104-218 the per-sampler update).  The reference runs these loops in
// JavaScript, where every product and sum is a double and every value stored into a
// Float32Array is rounded to float; this kernel forms the same values from the same operands in
// the same order in double precision, rounds at the same points, and is built without
// floating-point contraction, so its outputs are bit-identical to the reference's on equal
// inputs.  Elementwise and HBM-bound: per element it reads x, v (+ v_uncond, old, old_d, eps)
// and writes x (+ den, old, old_d).

#include <algorithm>

#include "common.h"
#include "internal.h"

namespace anima {

namespace {

// o = a x + b y, as `a * x[i] + b * y[i]` stored into a Float32Array
__device__ __forceinline__ float axpby(double a, float x, double b, float y) {
  return (float)(a * (double)x + b * (double)y);
}

__global__ __launch_bounds__(256) void sampler_step_kernel(anima_sampler_desc d) {
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < d.n; j += (int64_t)gridDim.x * 256) {
    float v = d.v[j];
    if (d.v_uncond) {  // vn[j] + cfg * (v[j] - vn[j])
      const double vn = d.v_uncond[j];
      v = (float)(vn + d.cfg * ((double)v - vn));
    }
    const float x = d.x[j];
    const float den = (float)((double)x - d.sigma * (double)v);  // xin[j] - sigma * v[j]
    if (d.den_out) d.den_out[j] = den;
    float xn;
    if (d.final_step) {
      xn = den;
    } else if (d.kind == ANIMA_SAMPLER_EULER) {
      xn = axpby(d.c[0], x, d.c[1], den);
    } else if (d.kind == ANIMA_SAMPLER_EULER_A) {
      const float t = axpby(d.c[0], x, d.c[1], den);
      xn = (float)(d.c[2] * (double)t + (double)d.eps[j] * d.c[3]);  // k * x[j] + eps[j] * renoise
    } else if (d.kind == ANIMA_SAMPLER_DPMPP_2M) {
      const float dd = d.stage ? axpby(d.c[2], den, d.c[3], d.old[j]) : den;
      xn = axpby(d.c[0], x, d.c[1], dd);
    } else {  // ANIMA_SAMPLER_ER_SDE
      xn = axpby(d.c[0], x, d.c[1], den);
      if (d.stage >= 2) {
        const float dD = axpby(d.c[2], den, d.c[3], d.old[j]);
        xn = (float)((double)xn + d.c[4] * (double)dD);  // x[j] += c2 * dD[j]
        if (d.stage >= 3) {
          const float dU = axpby(d.c[5], dD, d.c[6], d.old_d[j]);
          xn = (float)((double)xn + d.c[7] * (double)dU);
        }
        d.old_d[j] = dD;
      }
      if (d.eps) xn = (float)((double)xn + d.c[8] * (double)d.eps[j] * d.c[9]);  // alphaT * eps[j] * nz
    }
    d.x[j] = xn;
    if (d.old) d.old[j] = den;
  }
}

}  // namespace

int sampler_step_launch(anima_ctx* c, const anima_sampler_desc* d) {
  if (!d) return fail(c, ANIMA_E_ARG, "anima_sampler_step: null descriptor");
  if (d->kind < ANIMA_SAMPLER_EULER || d->kind > ANIMA_SAMPLER_ER_SDE)
    return fail(c, ANIMA_E_ARG, "anima_sampler_step: unknown sampler kind %d", d->kind);
  if (d->n < 0) return fail(c, ANIMA_E_ARG, "anima_sampler_step: n=%lld", (long long)d->n);
  if (!d->x || !d->v) return fail(c, ANIMA_E_ARG, "anima_sampler_step: null x or v");
  if (!d->final_step) {
    const bool needs_eps = d->kind == ANIMA_SAMPLER_EULER_A;
    if (needs_eps && !d->eps) return fail(c, ANIMA_E_ARG, "anima_sampler_step: euler_a needs eps");
    if (d->kind == ANIMA_SAMPLER_DPMPP_2M && d->stage && !d->old)
      return fail(c, ANIMA_E_ARG, "anima_sampler_step: dpmpp_2m after the first step needs old");
    if (d->kind == ANIMA_SAMPLER_ER_SDE) {
      if (d->stage < 1 || d->stage > 3) return fail(c, ANIMA_E_ARG, "anima_sampler_step: er_sde stage %d", d->stage);
      if (d->stage >= 2 && (!d->old || !d->old_d))
        return fail(c, ANIMA_E_ARG, "anima_sampler_step: er_sde stage %d needs old and old_d", d->stage);
    }
  }
  if (d->n == 0) return ANIMA_OK;
  const int nb = 4 + (d->v_uncond ? 4 : 0) + (d->den_out ? 4 : 0) + (d->old ? 8 : 0) + (d->old_d ? 8 : 0) + (d->eps ? 4 : 0);
  Launch lc(c, "sampler_step", 0.0, (double)d->n * (8 + nb));
  const unsigned grid = (unsigned)std::min<int64_t>((d->n + 255) / 256, 8192);
  hipLaunchKernelGGL(sampler_step_kernel, dim3(grid), dim3(256), 0, c->stream, *d);
  return lc.end();
}

}  // namespace anima
