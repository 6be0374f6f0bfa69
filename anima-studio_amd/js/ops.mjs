// Tensor ops with the signatures of the reference's app/gpu/ops.js, dispatched to the gfx950
// kernels of libanima.so through the N-API addon.  Activations are f32 Tensors (row-major).
//
// Extensions beyond the reference interface (all optional arguments):
//   attention: B / qBatch / kBatch / vBatch / oBatch (batched CFG), kvLen (per-batch valid keys),
//              qNorm / kNorm / cs (q/k RMSNorm + RoPE fused into the attention loads), precision.
//   linear:    opts.xq = { q, s } per-token int8 activations (layernormModQ / quantRows); with a
//              LoRA on a quantized weight the fp32 rotated input opts.xr is needed as well.
//   layernormModQ: LayerNorm + adaLN + ConvRot + per-token int8 in one pass.

import { native } from "./gpu.mjs";

const KIND = { bf16: 0, i8: 1, w4: 2, f32: 3 };
const ACT = { none: 0, gelu: 1, silu: 2 };
const EW = { silu_mul: 0, add: 1, silu: 2, copy: 3 };
const ptr = (t) => (t ? (typeof t === "number" ? t : t.buf) : 0);

export const needsRotation = (W) => W.kind === "i8" || W.kind === "w4";

// ConvRot input rotation (ops.js:38-44).
export function rotate(gpu, x) {
  const y = gpu.empty(x.shape);
  native.hadamard(gpu.ctx, x.buf, y.buf, x.size);
  return y;
}

// Per-token int8 quantization of rows [M, K] (optionally ConvRot-rotating first).
export function quantRows(gpu, x, K, rotateFirst) {
  const M = x.size / K;
  const q = gpu.empty([M, K], "i8");
  const s = gpu.empty([M]);
  native.quantRows(gpu.ctx, x.buf, M, K, rotateFirst ? 1 : 0, q.buf, s.buf);
  return { q, s, release() { q.release(); s.release(); } };
}

function weightArg(W) {
  if (!(W.kind in KIND)) throw new Error(`unsupported weight kind ${W.kind}`);
  return { kindId: KIND[W.kind], N: W.N, K: W.K, buf: ptr(W.buf), scale: ptr(W.scale), srel: ptr(W.srel),
    codebook: ptr(W.codebook), bias: ptr(W.bias) };
}

// y = x @ W^T (+ bias) (act) (ops.js:48-66).  Quantized weights take the ConvRot-rotated input
// `xr` when given, else rotate x here; the activations are quantized per token (W8A8).
// opts.out + opts.resid: out += (gate[gOff + n] *) y in place.
export function linear(gpu, x, W, opts) {
  const o = opts || {};
  const M = o.M !== undefined ? o.M : (o.xq ? o.xq.s.size : x.size / W.K);
  // LoRAs: delta = sum_i scale_i B_i (A_i x_in), added in the epilogue before act / gate
  // (ops.js:55-62); x_in is the rotated input for quantized weights (A was rotated at load).
  let delta = null, tmp = null;
  if (W.lora && W.lora.length) {
    let xin = x;
    if (needsRotation(W)) {
      if (o.xr) xin = o.xr;
      else if (x) xin = tmp = rotate(gpu, x);
      else throw new Error(`${W.name || "linear"}: a LoRA on a quantized weight needs the fp32 input (x or opts.xr)`);
    }
    delta = loraDelta(gpu, xin, W, M);
  }
  const out = o.out || gpu.empty([M, W.N]);
  const d = { M, out: out.buf, ldc: o.ldc || 0, alpha: o.alpha || 0, act: ACT[o.act || "none"],
    epilogue: o.resid ? (o.gate ? 2 : 1) : 0, gate: ptr(o.gate), gOff: o.gOff || 0, accOut: ptr(o.accOut),
    add: delta ? delta.buf : 0, ldAdd: delta ? W.N : 0 };
  if (needsRotation(W) && o.xq) {
    d.xq = o.xq.q.buf;
    d.xs = o.xq.s.buf;
  } else if (needsRotation(W)) {
    d.x = (o.xr || x).buf;
    d.xRotated = o.xr ? 1 : 0;
  } else {
    d.x = x.buf;
    d.ldx = o.ldx || 0;
  }
  const w = weightArg(W);
  if (o.bias) w.bias = ptr(o.bias);
  native.linear(gpu.ctx, w, d);
  if (delta) delta.release();
  if (tmp) tmp.release();
  return out;
}

// [M, W.N] low-rank update (ops.js:70-87).  Entries { A: [r, K] f32, B: [n, r] f32, r, scale,
// off, n }, off / n selecting the output columns (a slice of a stacked q/k/v weight).  A
// full-width entry, if any, initializes the delta; everything else accumulates into it.
function loraDelta(gpu, xin, W, M) {
  const D = gpu.empty([M, W.N]);
  const isFull = (e) => e.off === 0 && e.n === W.N;
  const entries = W.lora.slice().sort((a, b) => isFull(b) - isFull(a));
  let first = entries.some(isFull);
  if (!first) zero(gpu, D);
  for (const e of entries) {
    const t = linear(gpu, xin, { kind: "f32", N: e.r, K: W.K, buf: e.A }, { M });
    const store = first && isFull(e);
    linear(gpu, t, { kind: "f32", N: e.n, K: e.r, buf: e.B }, { M, out: D.view(e.off, [M, e.n]), ldc: W.N,
      alpha: e.scale, resid: !store });
    if (store) first = false;
    t.release();
  }
  return D;
}

export function zero(gpu, t) {
  native.zero(gpu.ctx, t.buf, t.size);
}

export function rmsnorm(gpu, x, weight, cols, eps, out) {
  const rows = x.size / cols;
  const y = out || gpu.empty(x.shape);
  native.rmsnorm(gpu.ctx, x.buf, ptr(weight), y.buf, rows, cols, eps === undefined ? 1e-6 : eps);
  return y;
}

// rotate: output is already ConvRot-rotated (input for quantized linears via { xr }) (ops.js:129-137)
export function layernormMod(gpu, x, mod, shiftOff, scaleOff, cols, rotateOut) {
  const rows = x.size / cols;
  const y = gpu.empty(x.shape);
  native.layernormMod(gpu.ctx, x.buf, ptr(mod), shiftOff, scaleOff, rows, cols, 1e-6, rotateOut ? 1 : 0, y.buf, 0, 0);
  return y;
}

// LayerNorm + adaLN + ConvRot + per-token int8: { q, s } for linear(..., { xq }); withRotated
// also returns the fp32 rotated rows as xr (the input of a LoRA side path).
export function layernormModQ(gpu, x, mod, shiftOff, scaleOff, cols, withRotated) {
  const rows = x.size / cols;
  const q = gpu.empty([rows, cols], "i8");
  const s = gpu.empty([rows]);
  const xr = withRotated ? gpu.empty([rows, cols]) : null;
  native.layernormMod(gpu.ctx, x.buf, ptr(mod), shiftOff, scaleOff, rows, cols, 1e-6, 1, xr ? xr.buf : 0, q.buf, s.buf);
  return { q, s, xr, release() { q.release(); s.release(); if (xr) xr.release(); } };
}

// In-place per-head RMSNorm + RoPE on the q and k parts of a fused QKV buffer [L, 3*H*D] (ops.js:140-145).
export function qkNormRope(gpu, qkv, qn, kn, cs, L, H, D) {
  native.qkNormRope(gpu.ctx, qkv.buf, L, H, D, 3 * H * D, ptr(qn), ptr(kn), ptr(cs), cs.sinOff, 1e-6);
}

// In-place rope on x viewed as [L, H, D] inside rows of `rowStride` starting at colOff (ops.js:148-152).
export function rope(gpu, x, cs, L, H, D, rowStride, colOff) {
  native.rope(gpu.ctx, x.buf, ptr(cs), L, H, D, cs.sinOff, rowStride || H * D, colOff || 0);
}

export function elementwise(gpu, op, a, b, out) {
  const y = out || gpu.empty(a.shape);
  native.elementwise(gpu.ctx, EW[op], a.buf, b ? b.buf : 0, y.buf, y.size);
  return y;
}

// Multi-head attention (ops.js:166-208), fused flash path on the matrix cores.
//  q: [Lq, ldq] with head h at column qOff + h*D; k, v: [Lk, ldk]/[Lk, ldv] with kv head
//  h/group at kOff/vOff + (h/group)*D.  Output [B*Lq, H*D].
export function attention(gpu, a) {
  const B = a.B || 1;
  const H = a.H, D = a.D;
  const o = a.out || gpu.empty([B * a.Lq, H * D]);
  native.attention(gpu.ctx, {
    B, Lq: a.Lq, Lk: a.Lk, H, D, group: a.group || 1,
    q: a.q.buf, k: a.k.buf, v: a.v.buf, o: o.buf,
    ldq: a.ldq, ldk: a.ldk, ldv: a.ldv, ldo: a.ldo || H * D,
    qOff: a.qOff || 0, kOff: a.kOff || 0, vOff: a.vOff || 0, oOff: a.oOff || 0,
    qBatch: a.qBatch !== undefined ? a.qBatch : a.Lq * a.ldq,
    kBatch: a.kBatch !== undefined ? a.kBatch : a.Lk * a.ldk,
    vBatch: a.vBatch !== undefined ? a.vBatch : a.Lk * a.ldv,
    oBatch: a.oBatch !== undefined ? a.oBatch : a.Lq * (a.ldo || H * D),
    scale: a.scale || 0, kvLen: a.kvLen || null, precision: a.precision === "fp32" ? 1 : 0,
    qNorm: ptr(a.qNorm), kNorm: ptr(a.kNorm), cs: ptr(a.cs), sinOff: a.cs ? a.cs.sinOff : 0, eps: 1e-6,
    causal: a.causal ? 1 : 0,
  });
  return o;
}

// VAE / text-encoder ops of the reference are outside the DiT attention path.
export function conv3x3() {
  throw new Error("conv3x3 (VAE) is not part of this build");
}
export function conv3x3Into() {
  throw new Error("conv3x3 (VAE) is not part of this build");
}
export function channelNorm() {
  throw new Error("channelNorm (VAE) is not part of this build");
}
