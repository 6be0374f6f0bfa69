// Tensor ops with the signatures of the reference's app/gpu/ops.js, dispatched to the gfx950
// kernels of libanima.so through the N-API addon.  Activations are f32 Tensors (row-major).
//
// Extensions beyond the reference interface (all optional arguments):
//   attention: B / qBatch / kBatch / vBatch / oBatch (batched CFG), kvLen (per-batch valid keys),
//              qNorm / kNorm / cs (q/k RMSNorm + RoPE fused into the attention loads), precision.
//   linear:    opts.xq = { q, s } per-token int8 activations (layernormModQ / quantRows); a LoRA
//              on a quantized weight reads them too (setLoraInput), or the fp32 input opts.xr / x.
//   layernormModQ: LayerNorm + adaLN + ConvRot + per-token int8 in one pass.

import { native } from "./gpu.mjs";

const KIND = { bf16: 0, i8: 1, w4: 2, f32: 3, f32s3: 4 };
const ACT = { none: 0, gelu: 1, silu: 2 };
const EW = { silu_mul: 0, add: 1, silu: 2, copy: 3 };
const ptr = (t) => (t ? (typeof t === "number" ? t : t.buf) : 0);

export const needsRotation = (W) => W.kind === "i8" || W.kind === "w4";

// The input of a quantized linear's LoRA A product.  "int8" (default): the per-token int8 rows
// the GEMM itself reads (opts.xq, ConvRot-rotated) against the rotated A (A H), so the LoRA sees
// the same activations as W and no fp32 copy of them is written.  "fp32": the fp32 input, rotated
// (opts.xr, with A H) or not (x, with A), as the reference's loraDelta takes it (ops.js:55-62).
let loraInputMode = "int8";
export function setLoraInput(mode) {
  if (mode !== "int8" && mode !== "fp32") throw new Error(`LoRA input "${mode}": "int8" or "fp32"`);
  loraInputMode = mode;
}
export const loraInput = () => loraInputMode;
// whether linear() runs W's LoRA A product from opts.xq (its fused factors with the rotated A)
export function loraReadsInt8(W) {
  const F = W.loraFused;
  return loraInputMode === "int8" && needsRotation(W) && !!(F && F.lora === W.lora && F.Ars);
}

// ConvRot input rotation (ops.js:38-44).
export function rotate(gpu, x) {
  const y = gpu.empty(x.shape);
  native.hadamard(gpu.ctx, x.buf, y.buf, x.size);
  return y;
}

// Per-token int8 quantization of rows [M, K] (optionally ConvRot-rotating first); bf16 rows (an
// attention output written with oBf16) are widened exactly first.
export function quantRows(gpu, x, K, rotateFirst, act) {
  const M = x.size / K;
  const q = gpu.empty([M, K], "i8");
  const s = gpu.empty([M]);
  if (x.dtype === "bf16") {
    if (act && act !== "none") throw new Error("quantRows: no activation on bf16 rows");
    native.quantRowsBf16(gpu.ctx, x.buf, M, K, rotateFirst ? 1 : 0, q.buf, s.buf);
  } else {
    native.quantRows(gpu.ctx, x.buf, M, K, rotateFirst ? 1 : 0, q.buf, s.buf, ACT[act || "none"]);
  }
  return { q, s, release() { q.release(); s.release(); } };
}

// A W4 weight turned into the int8 weight with the same products, in place (the object keeps its
// identity, so LoRA attachments and stacked views stay valid): the int8 grid replaces the codes
// (one byte per weight instead of half), s_channel stays the per-row scale.  Bit-identical
// linear results; the GEMM then skips the nibble unpack.
export function unpackW4(gpu, W) {
  if (W.kind !== "w4") return W;
  const grid = gpu.empty([W.N * W.K], "i8");
  native.weightUnpackW4(gpu.ctx, weightArg(W), grid.buf);
  for (const t of [W.buf, W.srel, W.codebook]) if (t && t.release) t.release();
  W.kind = "i8";
  W.buf = grid;
  W.srel = null;
  W.codebook = null;
  W.unpackedW4 = true;
  return W;
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
  // LoRAs: y += sum_i scale_i B_i (A_i x), after the bias and before act / gate (ops.js:55-62).
  // The reference feeds ConvRot layers' LoRAs the rotated input and a rotated A; since
  // (x H)(A H)^T = x A^T, the unrotated x and A are used when x is at hand (no rotation pass), and
  // the rotated pair (opts.xr, entry.Ar) only when the caller holds just the rotated input.
  const lora = W.lora && W.lora.length ? W.lora : null;
  // int8 LoRA input (setLoraInput): the A product over opts.xq with the rotated A
  const q8 = !!(lora && o.xq && loraReadsInt8(W));
  const rot = !q8 && !!(lora && needsRotation(W) && o.xr);
  const xin = q8 ? null : rot ? o.xr : x;
  if (lora && !q8 && !xin) throw new Error(`${W.name || "linear"}: a LoRA on a quantized weight needs its input (opts.xq, x or opts.xr)`);
  // Quantized weights with fused LoRA factors (fuseLora): one A product over the stacked A, and
  // the B product inside the GEMM's epilogue (no [M, N] delta).  Otherwise a plain store (no
  // activation, no residual) takes the LoRA products afterwards, accumulated straight into the
  // output, and other epilogues get them as a delta that the epilogue adds.
  const F = lora && W.loraFused && W.loraFused.lora === W.lora ? W.loraFused : null;
  if (F && rot && !F.Ar) throw new Error(`${W.name || "linear"}: LoRA entries without the rotated A for a rotated input`);
  const down = !F ? null
    : q8 ? linear(gpu, null, { kind: "f32s3", N: F.R, K: W.K, buf: F.Ars }, { M, xq: o.xq })
    : linear(gpu, xin, { kind: "f32s3", N: F.R, K: W.K, buf: rot ? F.Ars : F.As }, { M });
  const late = lora && !F && !o.resid && ACT[o.act || "none"] === 0;
  const delta = lora && !F && !late ? loraDelta(gpu, xin, W, M, rot) : null;
  const out = o.out || gpu.empty([M, W.N]);
  const d = { M, out: out.buf, ldc: o.ldc || 0, alpha: o.alpha || 0, act: ACT[o.act || "none"],
    epilogue: o.resid ? (o.gate ? 2 : 1) : 0, gate: ptr(o.gate), gOff: o.gOff || 0, accOut: ptr(o.accOut),
    add: delta ? delta.buf : 0, ldAdd: delta ? W.N : 0,
    loraXa: down ? down.buf : 0, ldLoraXa: down ? F.R : 0, loraB: F ? F.Bs.buf : 0, loraR: F ? F.Rb : 0,
    loraCols: F ? F.cols : 0 };
  if ((needsRotation(W) || W.kind === "f32s3") && o.xq) {
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
  if (late) loraInto(gpu, xin, W, M, out, o.ldc || W.N, false, rot);
  if (delta) delta.release();
  if (down) down.release();
  return out;
}

// The LoRA factors of a quantized weight for the GEMM epilogue (anima_linear_desc.lora_*): every
// entry's A (and A H) stacked into [R, K], and B as one matrix whose row n holds scale_e *
// B_e[n - off_e] in the columns of the ranks of the entries e covering column n (zeros elsewhere),
// so that y += (A x_in)^T-row times B-row sums sum_e scale_e B_e (A_e x_in) over those entries
// (ops.js:55-87).  When every entry covers one of the equal column blocks of a stacked weight
// (q / k / v with their own LoRAs), the ranks are kept per block (lora_cols): block b's entries
// fill ranks [b Rb, (b + 1) Rb) of the A stack, Rb their largest per-block sum rounded up to 16,
// and B is [N, Rb] with each row holding only its block's ranks; otherwise one block of R = the
// summed ranks rounded up to 16 (zero rows pad).  Built at attach time (B composed on the host
// from the device copies); owned by W, freed with its stack.
export function fuseLora(gpu, W) {
  releaseLoraFused(W);
  if (!W.lora || !W.lora.length || !needsRotation(W)) return null;
  const K = W.K, N = W.N, cols = W.lora[0].n;
  const blocked = N > cols && N % cols === 0 && cols % 16 === 0 && W.lora.every((e) => e.n === cols && e.off % cols === 0);
  const nb = blocked ? N / cols : 1, blk = (e) => (blocked ? e.off / cols : 0);
  const used = new Array(nb).fill(0), start = new Map();
  for (const e of W.lora) {
    start.set(e, used[blk(e)]);
    used[blk(e)] += e.r;
  }
  const Rb = Math.ceil(Math.max(...used) / 16) * 16, R = nb * Rb;
  const stack = (key) => {
    const A = gpu.empty([R, K]);
    if (used.some((u) => u < Rb)) zero(gpu, A);
    for (const e of W.lora) gpu.copy(A.at((blk(e) * Rb + start.get(e)) * K), e[key], e.r * K * 4);
    return A;
  };
  const A = stack("A"), Ar = W.lora.every((e) => e.Ar) ? stack("Ar") : null;
  const Bh = new Float32Array(N * Rb);
  for (const e of W.lora) {
    const b = new Float32Array(e.n * e.r), c0 = start.get(e);
    native.d2h(gpu.ctx, e.B.buf, b);
    for (let i = 0; i < e.n; i++)
      for (let j = 0; j < e.r; j++) Bh[(e.off + i) * Rb + c0 + j] = Math.fround(e.scale * b[i * e.r + j]);
  }
  const Bf = gpu.fromArray(Bh, [N, Rb]);
  W.loraFused = { A, Ar, As: splitPlanes(gpu, A, R * K), Ars: Ar ? splitPlanes(gpu, Ar, R * K) : null,
    Bs: splitPlanes(gpu, Bf, N * Rb), R, Rb, cols: blocked ? cols : 0, lora: W.lora };
  Bf.release();
  return W.loraFused;
}

export function releaseLoraFused(W) {
  const F = W.loraFused;
  if (F) for (const t of [F.A, F.Ar, F.As, F.Ars, F.Bs]) if (t) t.release();
  W.loraFused = null;
}

// The stacked QKV projection of a DiT self-attention with the attention's K / V operand
// preparation in the GEMM epilogue (anima_linear_qkv; app/models/dit.js:266-304 runs the linear,
// then qkNormRope, then the attention).  Returns { q: [M, H*128] fp32, kvPrep } for
// attention(gpu, { q, kvPrep, qNorm, cs, ... }); K is RMS-normed (kNorm) and rotated (cs) and the
// prepared bytes equal attentionPrepareKV of the plain linear's output.  Callers check
// qkvFusable first (int8 / W4 weights, tokens per image a multiple of 64).  linearQkv takes LoRAs
// too: their fused factors (fuseLora) with rank blocks of whole 256-column tiles, the A product
// over the int8 rows opts.xq (or the rotated fp32 rows opts.xr under setLoraInput("fp32")).  With
// rank-32 LoRAs the fused GEMM (at its register limit) is 0.2 ms per DiT step faster than the
// LoRA linear plus the attention's own K / V conversion (45.8 vs 46.0 ms).
export function qkvFusable(W, L, H) {
  if (W.lora && W.lora.length) {
    const F = W.loraFused;
    if (!(F && F.lora === W.lora && F.Ars && F.cols % 256 === 0)) return false;
  }
  return needsRotation(W) && L % 64 === 0 && H % 2 === 0 && W.N === 3 * H * 128;
}

// A Q-only projection for linearQkv(..., { prepareQ: true }): int8 / W4 weights of H * 128
// columns, tokens per image a multiple of 64.  linearQkv takes the LoRA factors here too (the
// attention then matches the LoRA linear + q_norm bit for bit), but that GEMM instance spills and
// measured slower than the LoRA linear + the attention's own Q load (46.2 vs 45.9 ms per rank-32
// DiT step), so LoRAs are declined.
export function qFusable(W, L, H) {
  return needsRotation(W) && !(W.lora && W.lora.length) && L % 64 === 0 && W.N === H * 128;
}

export function linearQkv(gpu, x, W, opts) {
  const o = opts || {};
  const { B, L, H } = o;
  const M = B * L;
  // opts.prepareQ: Q as the attention's prepared bf16 operand (opts.qNorm, the RoPE of opts.cs,
  // opts.scale) in qPrep instead of fp32 in q; a weight of H * 128 columns is then a Q-only
  // projection (no K / V)
  const qOnly = !!o.prepareQ && W.N === H * 128;
  const q = o.prepareQ ? null : gpu.empty([M, H * 128]);
  const qPrep = o.prepareQ ? gpu.empty([M * H * 128 * 2], "u8") : null;
  const bytes = qOnly ? 0 : native.attentionKvBytes(B, H, L, 0);
  const kvPrep = qOnly ? null : gpu.empty([bytes], "u8");
  const d = { M, out: q ? q.buf : 0, ldc: H * 128, alpha: o.alpha || 0 };
  if (o.xq) {
    d.xq = o.xq.q.buf;
    d.xs = o.xq.s.buf;
  } else {
    d.x = x.buf;
    d.xRotated = o.xRotated ? 1 : 0;
  }
  // LoRAs: the A product of the rotated input (x H)(A H)^T = x A^T (the int8 rows opts.xq, or the
  // fp32 rows opts.xr; setLoraInput), the B product in the epilogue
  const F = W.lora && W.lora.length ? W.loraFused : null;
  const q8 = !!(F && o.xq && loraReadsInt8(W));
  if (F && !q8 && !o.xr) throw new Error(`${W.name || "linearQkv"}: a LoRA needs the rotated input (opts.xq or opts.xr)`);
  const Wa = F ? { kind: "f32s3", N: F.R, K: W.K, buf: F.Ars } : null;
  const down = !F ? null : q8 ? linear(gpu, null, Wa, { M, xq: o.xq }) : linear(gpu, o.xr, Wa, { M });
  if (F) Object.assign(d, { loraXa: down.buf, ldLoraXa: F.R, loraB: F.Bs.buf, loraR: F.Rb, loraCols: F.cols });
  const w = weightArg(W);
  native.linearQkv(gpu.ctx, w, d, { B, L, H, kNorm: ptr(o.kNorm), cs: ptr(o.cs), sinOff: o.cs ? o.cs.sinOff : 0,
    eps: o.eps || 1e-6, kvPrep: ptr(kvPrep), kvPrepBytes: bytes, qNorm: ptr(o.qNorm), qPrep: ptr(qPrep),
    qScale: o.scale || 0 });
  if (down) down.release();
  return { q, qPrep, kvPrep };
}

// Adds (or, storeFirst, stores where it comes first over a column range) every LoRA entry's
// scale * B (A x_in) into columns [off, off + n) of out (row stride ldc) (ops.js:70-87).
// Entries { A: [r, K] f32, Ar: A H (ConvRot targets), B: [n, r] f32, r, scale, off, n }: the
// whole weight, or one part of a stacked q/k/v weight (parts are disjoint); rot selects Ar (x_in
// rotated).  With a stack (stackLora), all A x_in come from one product over the stacked A,
// reading x_in once.
function loraInto(gpu, xin, W, M, out, ldc, storeFirst, rot) {
  const S = W.loraStack && W.loraStack.lora === W.lora ? W.loraStack : null;
  // a matrix as a weight object: its three bf16 planes (kind f32s3, made by splitPlanes) when
  // present, else the fp32 matrix
  const mat = (f32, s3, N, K) => (s3 ? { kind: "f32s3", N, K, buf: s3 } : { kind: "f32", N, K, buf: f32 });
  const Aof = (e) => {
    if (rot && !e.Ar) throw new Error(`${W.name || "linear"}: LoRA entry without the rotated A for a rotated input`);
    return rot ? mat(e.Ar, e.Ars, e.r, W.K) : mat(e.A, e.As, e.r, W.K);
  };
  const down = S ? linear(gpu, xin, rot ? mat(S.Ar, S.Ars, S.R, W.K) : mat(S.A, S.As, S.R, W.K), { M }) : null;
  const covered = new Uint8Array(W.N);
  const isFull = (e) => e.off === 0 && e.n === W.N;
  const entries = W.lora.slice().sort((a, b) => isFull(b) - isFull(a));
  for (const e of entries) {
    const t = S ? down.view(S.roff.get(e), [M, e.r]) : linear(gpu, xin, Aof(e), { M });
    const store = storeFirst && covered[e.off] === 0;
    linear(gpu, t, mat(e.B, e.Bs, e.n, e.r), { M, ldx: S ? S.R : 0, out: out.view(e.off, [M, e.n]),
      ldc, alpha: e.scale, resid: !store });
    covered.fill(1, e.off, e.off + e.n);
    if (!S) t.release();
  }
  if (down) down.release();
}

// The [M, W.N] LoRA delta for the epilogue's add term.  The reference zeroes it (or stores the
// first full-width entry) and accumulates the rest; when the entries cover every column, storing
// the first entry over each column range gives the same sums (0 + v is v) without the clearing pass.
function loraDelta(gpu, xin, W, M, rot) {
  const D = gpu.empty([M, W.N]);
  const covered = new Uint8Array(W.N);
  for (const e of W.lora) covered.fill(1, e.off, e.off + e.n);
  const clear = covered.includes(0);
  if (clear) zero(gpu, D);
  loraInto(gpu, xin, W, M, D, W.N, !clear, rot);
  return D;
}

// Stacks the A (and, when every entry has one, Ar) matrices of W's LoRA entries into [sum r, K]
// tensors so that loraInto runs one A product per call (the entries share x_in).  Valid while
// W.lora is the same array; the stack is owned by W and freed by releaseLoraStack.  No-op for
// fewer than two entries.
export function stackLora(gpu, W) {
  releaseLoraStack(W);
  if (!W.lora || W.lora.length < 2) return null;
  const R = W.lora.reduce((s, e) => s + e.r, 0);
  const stack = (key) => {
    const A = gpu.empty([R, W.K]);
    let r0 = 0;
    for (const e of W.lora) {
      gpu.copy(A.at(r0 * W.K), e[key], e.r * W.K * 4);
      r0 += e.r;
    }
    return A;
  };
  const roff = new Map();
  let r0 = 0;
  for (const e of W.lora) {
    roff.set(e, r0);
    r0 += e.r;
  }
  const A = stack("A"), Ar = W.lora.every((e) => e.Ar) ? stack("Ar") : null;
  W.loraStack = { A, Ar, As: splitPlanes(gpu, A, R * W.K), Ars: Ar ? splitPlanes(gpu, Ar, R * W.K) : null, R, roff,
    lora: W.lora };
  return W.loraStack;
}

export function releaseLoraStack(W) {
  const S = W.loraStack;
  if (S) for (const t of [S.A, S.Ar, S.As, S.Ars]) if (t) t.release();
  W.loraStack = null;
}

// The three bf16 planes of an fp32 matrix of n values (anima_split3_bf16, the f32s3 weight form),
// or null when n % 8 != 0 (the fp32 kernels then take the matrix as it is).
export function splitPlanes(gpu, t, n) {
  if (n % 8) return null;
  const p = gpu.empty([3 * n], "u16");
  native.split3(gpu.ctx, t.buf || t, p.buf, n);
  return p;
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
// a.kvPrep: K/V converted beforehand by attentionPrepareKV (then a.k / a.v are not needed).
// a.qPrep: Q prepared by linearQkv(..., { prepareQ: true }) (then a.q, a.qNorm and the query side
// of a.cs are not needed; bf16 precision, D = 128).
// a.precision: "fp32" (default, the reference's arithmetic) or "bf16" (bf16 matrix-core operands,
// fp32 accumulation: the DiT's and the text encoder's choice).
// a.oBf16: the output as bf16 ([B * Lq, H * D], dtype "bf16"), the input of a quantized output
// projection (quantRows); bf16 precision on the flash kernels only.
export function attention(gpu, a) {
  const B = a.B || 1;
  const H = a.H, D = a.D;
  const o = a.out || gpu.empty([B * a.Lq, H * D], a.oBf16 ? "bf16" : "f32");
  native.attention(gpu.ctx, attnDesc(a, B, H, D, o, { kvPrep: ptr(a.kvPrep), kvPrepBytes: a.kvPrep ? a.kvPrep.bytes : 0 }));
  return o;
}

// The K/V half of attention on its own, into a new buffer for later attention(..., { kvPrep }):
// keys and values that serve many calls (the per-prompt cross-attention K/V) are converted once.
// a.q / a.out are still checked as for the full call (the query side is not computed).
export function attentionPrepareKV(gpu, a) {
  const B = a.B || 1;
  const H = a.H, D = a.D;
  const bytes = native.attentionKvBytes(B, H / (a.group || 1), a.Lk, precisionId(a));
  const prep = gpu.empty([bytes], "u8");
  const o = a.out || { buf: a.q.buf };
  native.attention(gpu.ctx, attnDesc(a, B, H, D, o, { prepareInto: prep.buf, kvPrepBytes: bytes }));
  return prep;
}

function precisionId(a) {
  const p = a.precision || "fp32";
  if (p !== "fp32" && p !== "bf16") throw new Error(`attention: unknown precision ${p}`);
  return p === "fp32" ? 1 : 0;
}

function attnDesc(a, B, H, D, o, extra) {
  return Object.assign({
    B, Lq: a.Lq, Lk: a.Lk, H, D, group: a.group || 1,
    q: a.q ? a.q.buf : 0, k: a.k ? a.k.buf : 0, v: a.v ? a.v.buf : 0, o: o.buf, qPrep: ptr(a.qPrep),
    ldq: a.ldq, ldk: a.ldk, ldv: a.ldv, ldo: a.ldo || H * D,
    qOff: a.qOff || 0, kOff: a.kOff || 0, vOff: a.vOff || 0, oOff: a.oOff || 0,
    qBatch: a.qBatch !== undefined ? a.qBatch : a.q ? a.Lq * a.ldq : 0,
    // no k / v (prepared K/V): their strides are not read
    kBatch: a.kBatch !== undefined ? a.kBatch : a.k ? a.Lk * a.ldk : 0,
    vBatch: a.vBatch !== undefined ? a.vBatch : a.v ? a.Lk * a.ldv : 0,
    oBatch: a.oBatch !== undefined ? a.oBatch : a.Lq * (a.ldo || H * D),
    scale: a.scale || 0, kvLen: a.kvLen || null, precision: precisionId(a),
    qNorm: ptr(a.qNorm), kNorm: ptr(a.kNorm), cs: ptr(a.cs), sinOff: a.cs ? a.cs.sinOff : 0, eps: 1e-6,
    causal: a.causal ? 1 : 0, oBf16: a.oBf16 ? 1 : 0,
  }, extra);
}

// 3x3 conv (pad 1) on an NHWC image [h*w, cin] -> [H*W, W.N] (ops.js:95-105); up = true reads the
// input through a 2x nearest upsample (the output is then 2h x 2w); `into`: out += conv (the residual
// of conv3x3Into).  W: bf16 OHWI weight [N, 9*cin] (+ W.bias).  opts.precision: "fp32" (default, the
// reference's arithmetic: activations enter the bf16 matrix cores as two bf16 terms) or "bf16";
// opts.B: images stacked along the rows.
export function conv3x3(gpu, x, W, h, w, up, into, opts) {
  const o = opts || {};
  if (W.kind !== "bf16") throw new Error(`conv3x3: ${W.name || "weight"} is ${W.kind}, expected bf16 (OHWI)`);
  const B = o.B || 1;
  const H = up ? 2 * h : h, Wd = up ? 2 * w : w;
  const cin = W.K / 9;
  const out = into || gpu.empty([B * H * Wd, W.N]);
  native.conv3x3(gpu.ctx, { B, H, W: Wd, cin, cout: W.N, up: up ? 1 : 0, x: x.buf, w: ptr(W.buf), bias: ptr(W.bias),
    out: out.buf, resid: into ? 1 : 0, precision: precisionId(o) });
  return out;
}

// out += conv3x3(x) (the residual connection fused into the epilogue; ops.js:106-109)
export function conv3x3Into(gpu, x, W, h, w, out, opts) {
  return conv3x3(gpu, x, W, h, w, false, out, opts);
}

// Wan VAE RMS_norm over channels (+ SiLU) (ops.js:119-126).
export function channelNorm(gpu, x, gamma, cols, silu) {
  const rows = x.size / cols;
  const y = gpu.empty(x.shape);
  native.channelNorm(gpu.ctx, x.buf, ptr(gamma), y.buf, rows, cols, silu ? 1 : 0);
  return y;
}
