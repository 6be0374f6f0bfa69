// Flow-matching sampling (app/samplers.js:1-218): the ComfyUI "simple" and "beta" sigma
// schedules, and the Euler, Euler-ancestral, DPM++ 2M and ER-SDE (VP, stage 3) updates.
//
// `SamplerPlan` computes, per step, the scalar coefficients of the update (the same expressions,
// in double precision, as the reference); the device loop (pipeline.mjs) hands them to
// anima_sampler_step, which applies them elementwise.  `sample` is the reference's host loop
// over Float32Arrays (same signature), built on the same plan and on `applyStep`, the host twin of
// the device kernel: both form every stored value from the same operands in the same order.

import { TorchGenerator } from "./rng.mjs";

export const timeShift = (shift, t) => (shift * t) / (1 + (shift - 1) * t);

// sigma(t) of the discrete flow model sampling: 1000 entries t = i / 1000, shifted, as float
function sigmaTable(shift) {
  const table = new Array(1000);
  for (let i = 0; i < 1000; i++) table[i] = Math.fround(timeShift(shift, (i + 1) / 1000));
  return table;
}

// "simple": steps evenly spaced (by 1000 / steps) down from the top of the table, then 0
export function simpleSigmas(steps, shift) {
  const table = sigmaTable(shift);
  const stride = 1000 / steps;
  const out = [];
  for (let k = 0; k < steps; k++) out.push(table[999 - Math.floor(k * stride)]);
  out.push(0);
  return out;
}

// ln Gamma(z): Lanczos approximation, g = 7, 9 coefficients (Numerical Recipes 3rd ed. 6.1)
const LANCZOS = [0.99999999999980993, 676.5203681218851, -1259.1392167224028, 771.32342877765313,
  -176.61502916214059, 12.507343278686905, -0.13857109526572012, 9.9843695780195716e-6, 1.5056327351493116e-7];
function lnGamma(z) {
  if (z < 0.5) return Math.log(Math.PI / Math.sin(Math.PI * z)) - lnGamma(1 - z); // reflection
  z -= 1;
  let a = LANCZOS[0];
  for (let k = 1; k < 9; k++) a += LANCZOS[k] / (z + k);
  const t = z + 7.5;
  return 0.5 * Math.log(2 * Math.PI) + (z + 0.5) * Math.log(t) - t + Math.log(a);
}

// continued fraction of the incomplete beta function, modified Lentz (Numerical Recipes 6.4)
function betaContinuedFraction(a, b, x) {
  const tiny = 1e-300;
  const clampTiny = (v) => (Math.abs(v) < tiny ? tiny : v);
  let c = 1;
  let d = 1 / clampTiny(1 - ((a + b) * x) / (a + 1));
  let h = d;
  for (let m = 1; m <= 300; m++) {
    const m2 = 2 * m;
    let num = (m * (b - m) * x) / ((a - 1 + m2) * (a + m2)); // even step
    d = 1 / clampTiny(1 + num * d);
    c = clampTiny(1 + num / c);
    h *= d * c;
    num = (-(a + m) * (a + b + m) * x) / ((a + m2) * (a + 1 + m2)); // odd step
    d = 1 / clampTiny(1 + num * d);
    c = clampTiny(1 + num / c);
    const delta = d * c;
    h *= delta;
    if (Math.abs(delta - 1) < 1e-15) break;
  }
  return h;
}

// regularized incomplete beta I_x(a, b), the continued fraction on the side where it converges
function betaCdf(x, a, b) {
  if (x <= 0) return 0;
  if (x >= 1) return 1;
  const lnFront = lnGamma(a + b) - lnGamma(a) - lnGamma(b) + a * Math.log(x) + b * Math.log(1 - x);
  if (x < (a + 1) / (a + b + 2)) return (Math.exp(lnFront) * betaContinuedFraction(a, b, x)) / a;
  return 1 - (Math.exp(lnFront) * betaContinuedFraction(b, a, 1 - x)) / b;
}

// inverse of I_x(a, b) by 100 bisection steps on [0, 1]
function betaPpf(p, a, b) {
  if (p <= 0) return 0;
  if (p >= 1) return 1;
  let lo = 0, hi = 1;
  for (let k = 0; k < 100; k++) {
    const mid = (lo + hi) / 2;
    if (betaCdf(mid, a, b) < p) lo = mid;
    else hi = mid;
  }
  return (lo + hi) / 2;
}

// "beta" (alpha = beta = 0.6): table indices round(999 * ppf(1 - k / steps)), repeated indices
// dropped (so fewer than `steps` steps can come back), then 0
export function betaSigmas(steps, shift, alpha = 0.6, beta = 0.6) {
  const table = sigmaTable(shift);
  const out = [];
  let prev = -1;
  for (let k = 0; k < steps; k++) {
    const t = Math.round(betaPpf(1 - k / steps, alpha, beta) * 999);
    if (t !== prev) out.push(table[t]);
    prev = t;
  }
  out.push(0);
  return out;
}

export const SCHEDULERS = { simple: simpleSigmas, beta: betaSigmas };

export const SAMPLER_KIND = { euler: 0, euler_a: 1, dpmpp_2m: 2, er_sde: 3 };

const ER_SDE_POINTS = 200; // Riemann points of the ER-SDE integrals
const erScaler = (v) => v * (Math.exp(Math.pow(v, 0.3)) + 10);

// Per-run coefficients of one sampler over a sigma schedule.  step(i) returns
// { kind, sigma, final, stage, noise, c } in the layout of anima_sampler_desc: sigma is the value
// the denoiser is called with, noise whether this step draws torch.randn(n) (in order, from the
// sampler's own generator).
export class SamplerPlan {
  constructor(name, sigmas, shift = 3) {
    if (!(name in SAMPLER_KIND)) throw new Error(`unknown sampler ${name}`);
    this.name = name;
    this.kind = SAMPLER_KIND[name];
    this.sigmas = sigmas;
    this.steps = sigmas.length - 1;
    if (name === "er_sde") {
      const sg = sigmas.slice();
      if (sg[0] >= 1) sg[0] = Math.fround(timeShift(shift, 1 - 1e-4));
      this.sg = sg;
      this.lam = sg.map((v) => (v === 0 ? 0 : v / (1 - v))); // sigma / alpha
    }
  }

  sigmaAt(i) {
    return this.sg ? this.sg[i] : this.sigmas[i];
  }

  step(i) {
    const c = new Array(10).fill(0);
    const out = { kind: this.kind, sigma: this.sigmaAt(i), final: false, stage: 0, noise: false, c };
    const s = this.sigmas[i], s1 = this.sigmas[i + 1];
    if (this.name === "euler") {
      if (s1 === 0) out.final = true;
      else {
        c[0] = s1 / s;
        c[1] = 1 - s1 / s;
      }
    } else if (this.name === "euler_a") { // rectified-flow ancestral step, eta = 1
      if (s1 === 0) out.final = true;
      else {
        const sDown = s1 * (s1 / s);
        const aNext = 1 - s1;
        const aDown = 1 - sDown;
        const renoise = Math.sqrt(s1 * s1 - (sDown * sDown * aNext * aNext) / (aDown * aDown));
        const r = sDown / s;
        c[0] = r;
        c[1] = 1 - r;
        c[2] = aNext / aDown;
        c[3] = renoise;
        out.noise = true;
      }
    } else if (this.name === "dpmpp_2m") {
      out.stage = i > 0 ? 1 : 0;
      if (s1 === 0) out.final = true;
      else {
        const lt = (v) => -Math.log(v);
        const h = lt(s1) - lt(s);
        c[0] = s1 / s;
        c[1] = -Math.expm1(-h);
        if (i > 0) {
          const r = (lt(s) - lt(this.sigmas[i - 1])) / h;
          c[2] = 1 + 1 / (2 * r);
          c[3] = -1 / (2 * r);
        }
      }
    } else { // er_sde
      const sg = this.sg, lam = this.lam;
      out.stage = Math.min(3, i + 1);
      if (sg[i + 1] === 0) out.final = true;
      else {
        const ls = lam[i], lt = lam[i + 1];
        const aS = sg[i] / ls, aT = sg[i + 1] / lt;
        const r = erScaler(lt) / erScaler(ls);
        c[0] = (aT / aS) * r;
        c[1] = aT * (1 - r);
        if (out.stage >= 2) {
          const dt = lt - ls;
          const h = -dt / ER_SDE_POINTS;
          let s0 = 0, s1w = 0;
          for (let p = 0; p < ER_SDE_POINTS; p++) {
            const pos = lt + p * h;
            const sc = erScaler(pos);
            s0 += 1 / sc;
            s1w += (pos - ls) / sc;
          }
          s0 *= h;
          s1w *= h;
          c[2] = 1 / (ls - lam[i - 1]);
          c[3] = -1 / (ls - lam[i - 1]);
          c[4] = aT * (dt + s0 * erScaler(lt));
          if (out.stage >= 3) {
            c[5] = 2 / (ls - lam[i - 2]);
            c[6] = -2 / (ls - lam[i - 2]);
            c[7] = aT * ((dt * dt) / 2 + s1w * erScaler(lt));
          }
        }
        const nz = Math.sqrt(Math.max(0, lt * lt - ls * ls * r * r));
        if (nz > 0) {
          out.noise = true;
          c[8] = aT;
          c[9] = nz;
        }
      }
    }
    return out;
  }
}

// Host twin of anima_sampler_step's update (given den): returns the new x; `state` carries
// old / oldD between steps.
export function applyStep(st, x, den, state, eps) {
  const n = x.length, c = st.c;
  if (st.final) {
    state.old = den;
    return den;
  }
  const o = new Float32Array(n);
  if (st.kind === 0) {
    for (let j = 0; j < n; j++) o[j] = c[0] * x[j] + c[1] * den[j];
  } else if (st.kind === 1) {
    for (let j = 0; j < n; j++) o[j] = c[0] * x[j] + c[1] * den[j];
    for (let j = 0; j < n; j++) o[j] = c[2] * o[j] + eps[j] * c[3];
  } else if (st.kind === 2) {
    let dd = den;
    if (st.stage) {
      dd = new Float32Array(n);
      for (let j = 0; j < n; j++) dd[j] = c[2] * den[j] + c[3] * state.old[j];
    }
    for (let j = 0; j < n; j++) o[j] = c[0] * x[j] + c[1] * dd[j];
  } else {
    for (let j = 0; j < n; j++) o[j] = c[0] * x[j] + c[1] * den[j];
    if (st.stage >= 2) {
      const dD = new Float32Array(n);
      for (let j = 0; j < n; j++) dD[j] = c[2] * den[j] + c[3] * state.old[j];
      for (let j = 0; j < n; j++) o[j] += c[4] * dD[j];
      if (st.stage >= 3) {
        const dU = new Float32Array(n);
        for (let j = 0; j < n; j++) dU[j] = c[5] * dD[j] + c[6] * state.oldD[j];
        for (let j = 0; j < n; j++) o[j] += c[7] * dU[j];
      }
      state.oldD = dD;
    }
    if (eps) for (let j = 0; j < n; j++) o[j] += c[8] * eps[j] * c[9];
  }
  state.old = den;
  return o;
}

// The reference's sampling loop (app/samplers.js:104): denoise(x, sigma, i) returns the x0
// prediction; x and the result are Float32Arrays.
export async function sample(name, denoise, x, sigmas, opts) {
  const o = opts || {};
  const plan = new SamplerPlan(name, sigmas, o.shift === undefined ? 3 : o.shift);
  const gen = new TorchGenerator(o.seed || 0); // the sampler's own noise generator
  const state = { old: null, oldD: null };
  for (let i = 0; i < plan.steps; i++) {
    const st = plan.step(i);
    const den = await denoise(x, st.sigma, i);
    x = applyStep(st, x, den, state, st.noise ? gen.randn(x.length) : null);
    if (o.onStep) await o.onStep(i, x, den);
  }
  return x;
}
