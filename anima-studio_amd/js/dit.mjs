// Anima DiT (Cosmos-Predict2 MiniTrainDIT, 28 blocks) on the gfx950 op layer.
// Restates the call order of app/models/dit.js (timeCond 196-225, prepareContext 232-249,
// forward 253-325) with two MI355X-side changes:
//   * CFG runs as one batched B=2 pass (cond + uncond) instead of two B=1 passes
//     (app/pipeline.js:260-265); each batch element attends to its own cached context K/V.
//   * Quantized linears run W8A8: LayerNorm + adaLN + ConvRot + per-token int8 are one kernel
//     (layernormModQ) feeding the int8-MFMA GEMM; q/k RMSNorm + RoPE are fused into attention.

import * as ops from "./ops.mjs";
import { concatLinears } from "./weights.mjs";
import { ditRopeTable, ropeTable, timestepEmbedding } from "./common.mjs";
import { native } from "./gpu.mjs";

const D = 2048;
const HEADS = 16;
const HD = 128;
const MLP = 8192;
const CTX_DIM = 1024;
const ADALN_RANK = 256;

function releaseAll(xs) {
  for (const x of xs) if (x && x.release) x.release();
}

// whether a quantized W's LoRA needs the fp32 rotated rows beside the int8 ones (its A product
// reads the int8 rows unless ops.setLoraInput("fp32"))
const wantsXr = (W) => !!(W.lora && W.lora.length) && !ops.loraReadsInt8(W);

// LayerNorm + adaLN for inputs that feed W: int8 { xq } when W is quantized (W8A8), else the
// fp32 modulated rows (normFor of app/models/dit.js:34-38).
function normFor(gpu, x, mod, W) {
  if (ops.needsRotation(W)) return { xq: ops.layernormModQ(gpu, x, mod, 0, D, D, wantsXr(W)) };
  return { n: ops.layernormMod(gpu, x, mod, 0, D, D, false) };
}

function project(gpu, nf, W, M, opts) {
  const o = Object.assign({ M }, opts || {});
  if (nf.xq) {
    o.xq = nf.xq;
    if (nf.xq.xr) o.xr = nf.xq.xr;
  }
  return ops.linear(gpu, nf.n || null, W, o);
}

// The attention output projection with its gated residual into x: a bf16 output (attention's
// oBf16) is quantized here, the form the int8 / W4 GEMM reads, otherwise ops.linear quantizes the
// fp32 rows itself.
function outProject(gpu, a, W, M, x, mod) {
  if (a.dtype === "bf16") {
    const aq = ops.quantRows(gpu, a, D, true);
    ops.linear(gpu, null, W, { M, xq: aq, out: x, resid: true, gate: mod, gOff: 2 * D });
    aq.release();
  } else {
    ops.linear(gpu, a, W, { M, out: x, resid: true, gate: mod, gOff: 2 * D });
  }
}

// whether an attention may write bf16 O for the output projection W (quantized, and its LoRA if
// any reads the int8 rows)
const bf16Out = (W, precision) => precision === "bf16" && ops.needsRotation(W) && !wantsXr(W);

function releaseNorm(nf) {
  if (nf.xq) nf.xq.release();
  if (nf.n) nf.n.release();
}

// The self-attention input projection when q, k and v could not be stacked (the unstacked path of
// app/models/dit.js:274-288): three linears on the same modulated rows, written into the column
// slices of one [M, 3D] buffer (row stride 3D), so the attention with its fused q/k RMSNorm + RoPE
// reads them exactly as it reads the stacked GEMM's output.  The LayerNorm runs once per input
// form the parts need (int8 rows for quantized parts, fp32 rows for bf16 parts).
function projectParts(gpu, x, mod, Ws, M) {
  const quant = Ws.filter((W) => ops.needsRotation(W));
  const xq = quant.length ? ops.layernormModQ(gpu, x, mod, 0, D, D, quant.some(wantsXr)) : null;
  const n = quant.length < Ws.length ? ops.layernormMod(gpu, x, mod, 0, D, D, false) : null;
  const qkv = gpu.empty([M, 3 * D]);
  Ws.forEach((W, j) => {
    if (W.N !== D || W.K !== D) throw new Error(`self-attention part ${j}: [${W.N}, ${W.K}], expected [${D}, ${D}]`);
    const o = { M, out: qkv.view(j * D, [M, D]), ldc: 3 * D };
    if (ops.needsRotation(W)) {
      o.xq = xq;
      if (xq.xr) o.xr = xq.xr;
    }
    ops.linear(gpu, ops.needsRotation(W) ? null : n, W, o);
  });
  releaseAll([xq, n]);
  return qkv;
}

// out[g] += B_g (A_g x_g) for the G parts of a grouped modulation LoRA stage (modLoraPlan): x_g =
// x + g * xStride (xStride 0: one row shared by every part), out[g] = out's g-th st.n-slice; the
// scales are folded into B_g.
function loraGrouped(gpu, st, x, xStride, out) {
  const t = gpu.empty([st.G * st.r]);
  if (xStride === 0) native.gemvGroupedF32(gpu.ctx, 1, st.G * st.r, st.K, x.buf, 0, st.A.buf, 0, t.buf, 0, 1, 0);
  else native.gemvGroupedF32(gpu.ctx, st.G, st.r, st.K, x.buf, xStride, st.A.buf, st.r * st.K, t.buf, st.r, 1, 0);
  native.gemvGroupedF32(gpu.ctx, st.G, st.n, st.r, t.buf, st.r, st.B.buf, st.n * st.r, out.buf, st.n, 1, 1);
  t.release();
}

// out (an M = 1 row) += scale * B (A x) for one LoRA entry of a linear whose product runs outside
// ops.linear (the grouped modulation GEMV); x is that linear's input row.
function loraPart(gpu, x, e, out) {
  const t = ops.linear(gpu, x, { kind: "f32", N: e.r, K: x.size, buf: e.A }, { M: 1 });
  ops.linear(gpu, t, { kind: "f32", N: e.n, K: e.r, buf: e.B }, { M: 1, out, alpha: e.scale, resid: true });
  t.release();
}

export class AnimaDiT {
  // From a safetensors checkpoint in the web-asset layout (app/models/dit.js:82-129).
  static load(gpu, st, nBlocks) {
    const m = new AnimaDiT(gpu);
    const attn = (p, o) => ({
      q: st.linear(gpu, p + "q_proj."), k: st.linear(gpu, p + "k_proj."), v: st.linear(gpu, p + "v_proj."),
      o: st.linear(gpu, p + o + "."), qn: st.vector(gpu, p + "q_norm.weight"), kn: st.vector(gpu, p + "k_norm.weight"),
    });
    m.xEmbed = st.linear(gpu, "x_embedder.proj.1.");
    m.t1 = st.linear(gpu, "t_embedder.1.linear_1.");
    m.t2 = st.linear(gpu, "t_embedder.1.linear_2.");
    m.tNorm = st.vector(gpu, "t_embedding_norm.weight");
    m.blocks = [];
    const n = nBlocks || 28;
    for (let i = 0; i < n; i++) {
      const p = `blocks.${i}.`;
      const mod = (nm) => [st.linear(gpu, p + nm + ".1."), st.linear(gpu, p + nm + ".2.")];
      const self = attn(p + "self_attn.", "output_proj");
      // one [3D, D] GEMM instead of three; null when the formats cannot be stacked (W4 parts with
      // different codebooks, mixed kinds): then q, k and v stay separate (dit.js:112-114)
      self.qkv = concatLinears(gpu, [self.q, self.k, self.v]);
      if (self.qkv) {
        delete self.q; delete self.k; delete self.v;
      }
      m.blocks.push({
        modSelf: mod("adaln_modulation_self_attn"), modCross: mod("adaln_modulation_cross_attn"),
        modMlp: mod("adaln_modulation_mlp"), self, cross: attn(p + "cross_attn.", "output_proj"),
        l1: st.linear(gpu, p + "mlp.layer1."), l2: st.linear(gpu, p + "mlp.layer2."),
      });
    }
    m.finalMod = [st.linear(gpu, "final_layer.adaln_modulation.1."), st.linear(gpu, "final_layer.adaln_modulation.2.")];
    m.finalLinear = st.linear(gpu, "final_layer.linear.");
    m.fuseModulation();
    return m;
  }

  // Seeded random-init weights of the same architecture (SyntheticWeights).  opts.fuse = false
  // keeps the per-linear adaLN modulation path.
  static synthetic(gpu, src, opts) {
    const m = new AnimaDiT(gpu);
    const bf = (name, N, K) => src.bf16Linear(gpu, name, N, K, 1.0);
    m.xEmbed = bf("x_embedder.proj.1", D, 68);
    m.t1 = bf("t_embedder.1.linear_1", D, D);
    m.t2 = bf("t_embedder.1.linear_2", 3 * D, D);
    m.tNorm = src.vector(gpu, "t_embedding_norm.weight", D);
    m.blocks = [];
    for (let i = 0; i < src.nBlocks; i++) {
      const p = `blocks.${i}.`;
      const mod = (nm) => [bf(p + nm + ".1", ADALN_RANK, D), src.bf16Linear(gpu, p + nm + ".2", 3 * D, ADALN_RANK, 0.1)];
      const L = (nm, N, K) => src.blockLinear(gpu, p + nm, N, K, i);
      m.blocks.push({
        modSelf: mod("adaln_modulation_self_attn"), modCross: mod("adaln_modulation_cross_attn"),
        modMlp: mod("adaln_modulation_mlp"),
        // the stacked q/k/v carry their parts' module names (as concatLinears' output), for LoRAs
        self: { qkv: Object.assign(L("self_attn.qkv", 3 * D, D), { parts: ["q_proj", "k_proj", "v_proj"].map((nm, j) =>
          ({ name: p + "self_attn." + nm, off: j * D, n: D })) }), o: L("self_attn.output_proj", D, D),
          qn: src.vector(gpu, p + "self_attn.q_norm.weight", HD), kn: src.vector(gpu, p + "self_attn.k_norm.weight", HD) },
        cross: { q: L("cross_attn.q_proj", D, D), k: L("cross_attn.k_proj", D, CTX_DIM), v: L("cross_attn.v_proj", D, CTX_DIM),
          o: L("cross_attn.output_proj", D, D),
          qn: src.vector(gpu, p + "cross_attn.q_norm.weight", HD), kn: src.vector(gpu, p + "cross_attn.k_norm.weight", HD) },
        l1: L("mlp.layer1", MLP, D), l2: L("mlp.layer2", D, MLP),
      });
    }
    m.finalMod = [bf("final_layer.adaln_modulation.1", ADALN_RANK, D), src.bf16Linear(gpu, "final_layer.adaln_modulation.2", 2 * D, ADALN_RANK, 0.1)];
    m.finalLinear = bf("final_layer.linear", 64, D);
    if (!opts || opts.fuse !== false) m.fuseModulation();
    return m;
  }

  constructor(gpu) {
    this.gpu = gpu;
    this.ropeCache = new Map(); // "HpxWp" -> device RoPE table; depends only on the token grid
    this.modFused = null;
    this.modPlan = null; // grouped LoRA products of the fused modulation (modLoraPlan)
    // attention precision: bf16 matrix-core operands with fp32 accumulation ("fp32": the fp32-MFMA
    // kernels, the reference's arithmetic); prepareContext records the one its K/V were made for
    this.precision = "bf16";
    // self-attention K / V prepared in the QKV GEMM's epilogue where the weight allows
    // (ops.qkvFusable); false runs the linear and the attention's own K / V conversion
    this.fuseQkv = true;
  }

  // Converts every W4 block linear to its int8 grid once (ops.unpackW4): the GEMMs then run on the
  // int8 path with bit-identical results and no nibble unpack per call, at one byte per weight
  // (a load-time option for a device with the memory to spare; the packed form is the default).
  // Returns the number of linears converted.
  unpackW4() {
    let n = 0;
    for (const b of this.blocks) {
      const Ws = [b.self.qkv, b.self.q, b.self.k, b.self.v, b.self.o, b.cross.q, b.cross.k, b.cross.v, b.cross.o, b.l1, b.l2];
      for (const W of Ws) {
        if (W && W.kind === "w4") {
          ops.unpackW4(this.gpu, W);
          n++;
        }
      }
    }
    return n;
  }

  // The 3 * blocks + 1 adaLN modulation linears all read the same SiLU(t-embedding) (dit.js:205-
  // 222): their first stages are stacked into one [(3B+1)*256, 2048] weight (one GEMV) and the
  // blocks' second stages into one [3B*6144, 256] weight run as one grouped GEMV, with adaln_lora
  // added as a bias shared by every group (the same sum as the reference's lora + W2 h).  Only
  // for bias-free bf16 weights (the checkpoint format); otherwise the per-linear path stays.
  fuseModulation() {
    const first = [], second = [];
    for (const b of this.blocks) {
      first.push(b.modSelf[0], b.modCross[0], b.modMlp[0]);
      second.push(b.modSelf[1], b.modCross[1], b.modMlp[1]);
    }
    first.push(this.finalMod[0]);
    const ok = (ws) => ws.every((w) => w.kind === "bf16" && w.K === ws[0].K && w.N === ws[0].N && !w.bias);
    if (!ok(first) || !ok(second) || this.finalMod[1].kind !== "bf16" || this.finalMod[1].bias) return;
    this.modFused = { w1: concatLinears(this.gpu, first), w2: concatLinears(this.gpu, second), final2: this.finalMod[1] };
    for (const b of this.blocks) { delete b.modSelf; delete b.modCross; delete b.modMlp; }
    this.finalMod = null;
  }

  ropeTable(Hp, Wp) {
    const key = `${Hp}x${Wp}`;
    let t = this.ropeCache.get(key);
    if (!t) {
      t = ditRopeTable(this.gpu, Hp, Wp);
      this.ropeCache.set(key, t);
    }
    return t;
  }

  // Frees the device tables cached across forward calls and the grouped modulation LoRA plan (the
  // weights belong to their loader).
  releaseCaches() {
    for (const t of this.ropeCache.values()) t.release();
    this.ropeCache.clear();
    this.releaseModPlan();
  }

  // Everything that depends only on sigma (app/models/dit.js:196-225).
  timeCond(sigma) {
    const gpu = this.gpu;
    const t = gpu.fromArray(timestepEmbedding(sigma), [1, D]);
    const h = ops.linear(gpu, t, this.t1, { act: "silu" });
    const lora = ops.linear(gpu, h, this.t2); // adaln_lora [1, 6144]
    h.release();
    const emb = ops.rmsnorm(gpu, t, this.tNorm, D);
    t.release();
    const semb = ops.elementwise(gpu, "silu", emb);
    emb.release();
    if (this.modFused) {
      const { w1, w2, final2 } = this.modFused;
      const G = 3 * this.blocks.length, R = ADALN_RANK;
      const plan = this.modLoraPlan();
      // LoRAs on first stages: grouped (plan.s1) after the plain product, else inside ops.linear
      const h1 = ops.linear(gpu, semb, plan.s1 ? Object.assign({}, w1, { lora: null }) : w1); // [1, (G + 1) * 256]
      if (plan.s1) loraGrouped(gpu, plan.s1, semb, 0, h1);
      const all = gpu.empty([G, 3 * D]);
      native.linearGroupedBf16(gpu.ctx, G, 1, 3 * D, R, h1.buf, (G + 1) * R, R, w2.buf.buf, 3 * D * R, lora.buf, 0,
        all.buf, 3 * D, 3 * D);
      const final = gpu.empty([1, 2 * D]);
      native.linearGroupedBf16(gpu.ctx, 1, 1, 2 * D, R, h1.at(G * R), R, 0, final2.buf.buf, 0, lora.buf, 0, final.buf,
        2 * D, 0);
      // LoRAs on second stages: part j of w2 is group j, which reads h1's j-th 256-slice
      if (plan.s2) loraGrouped(gpu, plan.s2, h1, R, all);
      else if (w2.lora) for (const e of w2.lora) loraPart(gpu, h1.view((e.off / (3 * D)) * R, [1, R]), e, all.view(e.off, [1, e.n]));
      if (final2.lora) for (const e of final2.lora) loraPart(gpu, h1.view(G * R, [1, R]), e, final.view(e.off, [1, e.n]));
      h1.release();
      semb.release();
      lora.release();
      return this.timeCondFrom([all, final], true);
    }
    const mod = (ws, n) => {
      const out = gpu.empty([1, n]);
      ops.elementwise(gpu, "copy", lora, null, out); // the first n entries
      const hh = ops.linear(gpu, semb, ws[0]);
      ops.linear(gpu, hh, ws[1], { out, resid: true });
      hh.release();
      return out;
    };
    const parts = [];
    for (const b of this.blocks) parts.push(mod(b.modSelf, 3 * D), mod(b.modCross, 3 * D), mod(b.modMlp, 3 * D));
    parts.push(mod(this.finalMod, 2 * D));
    semb.release();
    lora.release();
    return this.timeCondFrom(parts, false);
  }

  // The LoRA products of the fused modulation as grouped fp32 GEMVs (anima_gemv_grouped_f32): per
  // stage (w1: the first stages, parts of 256 columns; w2: the second stages, parts of 3D columns,
  // part j reading h1's j-th 256-slice) one A product and one B product over all its entries,
  // instead of two launches per entry.  A stage qualifies when its entries have one rank and at
  // most one entry per part: the A matrices are stacked per part (zero rows for parts without an
  // entry) and the B matrices likewise, each scaled by its entry's scale.  Built once per LoRA
  // attachment (W.lora is replaced on every attach); { s1, s2 } with null for a stage without
  // entries or of another layout (that stage keeps the per-entry products).
  modLoraPlan() {
    const { w1, w2 } = this.modFused;
    const p = this.modPlan;
    if (p && p.l1 === w1.lora && p.l2 === w2.lora) return p;
    this.releaseModPlan();
    const gpu = this.gpu;
    const stage = (W, partN) => {
      const es = W.lora || [];
      if (!es.length || W.K % 4) return null;
      const r = es[0].r, G = W.N / partN, seen = new Set();
      for (const e of es) {
        if (e.r !== r || r % 4 || e.n !== partN || e.off % partN || seen.has(e.off)) return null;
        seen.add(e.off);
      }
      const A = gpu.empty([G * r, W.K]);
      const Bh = new Float32Array(G * partN * r), b = new Float32Array(partN * r);
      if (es.length < G) ops.zero(gpu, A);
      for (const e of es) {
        const g = e.off / partN;
        gpu.copy(A.at(g * r * W.K), e.A, r * W.K * 4);
        native.d2h(gpu.ctx, e.B.buf, b);
        for (let i = 0; i < b.length; i++) Bh[g * b.length + i] = Math.fround(e.scale * b[i]);
      }
      return { G, r, K: W.K, n: partN, A, B: gpu.fromArray(Bh, [G * partN, r]) };
    };
    this.modPlan = { l1: w1.lora, l2: w2.lora, s1: stage(w1, ADALN_RANK), s2: stage(w2, 3 * D) };
    return this.modPlan;
  }

  releaseModPlan() {
    const p = this.modPlan;
    if (p) for (const st of [p.s1, p.s2]) if (st) releaseAll([st.A, st.B]);
    this.modPlan = null;
  }

  // A timeCond result over its tensors: fused, [all [3*blocks, 3D], final [1, 2D]] (blocks are
  // views into `all`); otherwise [self, cross, mlp per block..., final].  `parts` lists them in
  // that order (timeCondSlot / copyTimeCond).
  timeCondFrom(parts, fused) {
    let blocks;
    if (fused) {
      const all = parts[0];
      blocks = this.blocks.map((_, i) => ({
        self: all.view(3 * i * 3 * D, [1, 3 * D]), cross: all.view((3 * i + 1) * 3 * D, [1, 3 * D]),
        mlp: all.view((3 * i + 2) * 3 * D, [1, 3 * D]),
      }));
    } else {
      blocks = this.blocks.map((_, i) => ({ self: parts[3 * i], cross: parts[3 * i + 1], mlp: parts[3 * i + 2] }));
    }
    return {
      blocks, final: parts[parts.length - 1], parts, fused,
      release() {
        releaseAll(parts);
      },
    };
  }

  // Uninitialized device tensors shaped like the timeCond result `like` (a fixed home for the
  // modulation vectors of a recorded forward, filled by copyTimeCond).
  timeCondSlot(like) {
    return this.timeCondFrom(like.parts.map((t) => this.gpu.empty(t.shape)), like.fused);
  }

  copyTimeCond(dst, src) {
    if (dst.parts.length !== src.parts.length) throw new Error("copyTimeCond: different timeCond layouts");
    dst.parts.forEach((t, i) => this.gpu.copy(t, src.parts[i], src.parts[i].bytes));
  }

  // Cross-attention K/V of every block for B prompts (app/models/dit.js:232-249): contexts are
  // stacked into one [B*Lk, 1024] buffer; per block k = RMSNorm(ctx Wk) (per head), v = ctx Wv,
  // each [B*Lk, 2048].  Takes ownership of the context tensors.
  prepareContext(ctxs) {
    const gpu = this.gpu;
    const B = ctxs.length;
    const Lk = ctxs[0].shape[0];
    const ctx = gpu.empty([B * Lk, CTX_DIM]);
    ctxs.forEach((c, b) => {
      if (c.shape[0] !== Lk) throw new Error("prepareContext: contexts must have the same length (pad to 512)");
      gpu.copy(ctx.at(b * Lk * CTX_DIM), c, Lk * CTX_DIM * 4);
      c.release();
    });
    const quant = this.blocks.some((b) => ops.needsRotation(b.cross.k));
    const xq = quant ? ops.quantRows(gpu, ctx, CTX_DIM, true) : null;
    // per block: k = RMSNorm(ctx Wk), v = ctx Wv, then converted once to the attention operand
    // layout (bf16 K rows, bf16 V^T) and kept; the fp32 k / v are released
    const kv = this.blocks.map((b) => {
      const k = ops.linear(gpu, ctx, b.cross.k, xq ? { xq, M: B * Lk } : { M: B * Lk });
      ops.rmsnorm(gpu, k, b.cross.kn, HD, 1e-6, k);
      const v = ops.linear(gpu, ctx, b.cross.v, xq ? { xq, M: B * Lk } : { M: B * Lk });
      const prep = ops.attentionPrepareKV(gpu, { q: k, k, v, B, Lq: Lk, Lk, H: HEADS, D: HD, ldq: D, ldk: D, ldv: D,
        precision: this.precision });
      releaseAll([k, v]);
      return { prep };
    });
    if (xq) xq.release();
    return {
      ctx, kv, Lk, B, precision: this.precision,
      release() {
        ctx.release();
        for (const e of kv) e.prep.release();
      },
    };
  }

  // Several prepared conditionings (prepareContext results, e.g. one per prompt from a cache) as
  // one batched conditioning, in the given order: per block, each part's prepared K plane and V^T
  // plane ([B][heads][Lkp][128] each) are copied side by side on the device.  The parts stay the
  // caller's; release() of the result frees only the copies.
  stackConds(conds) {
    const gpu = this.gpu;
    const Lk = conds[0].Lk, precision = conds[0].precision;
    for (const c of conds)
      if (c.Lk !== Lk || c.precision !== precision) throw new Error("stackConds: contexts must share Lk and precision");
    const B = conds.reduce((a, c) => a + c.B, 0);
    const kv = this.blocks.map((_, i) => {
      const prep = gpu.empty([conds.reduce((a, c) => a + c.kv[i].prep.bytes, 0)], "u8");
      const plane = prep.bytes / 2;
      let off = 0;
      for (const c of conds) {
        const src = c.kv[i].prep, half = src.bytes / 2;
        gpu.copy(prep.at(off), src.at(0), half);
        gpu.copy(prep.at(plane + off), src.at(half), half);
        off += half;
      }
      return { prep };
    });
    return {
      kv, Lk, B, precision,
      release() {
        for (const e of kv) e.prep.release();
      },
    };
  }

  // latents: B Float32Arrays [16, h, w]; cond: prepareContext(...) with the same B; tc: timeCond.
  // Returns B flow velocities [16, h, w] (app/models/dit.js:253-325).
  async forward(latents, h, w, cond, tc, onBlock) {
    const gpu = this.gpu;
    const B = latents.length;
    // latents go up as they are; the patch layout (dit.js:55-65) is built on the device
    const per = 16 * h * w;
    const host = new Float32Array(B * per);
    latents.forEach((lat, b) => {
      if (lat.length !== per) throw new Error(`forward: latent ${b} has ${lat.length} values, expected ${per}`);
      host.set(lat, b * per);
    });
    const lat = gpu.fromArray(host, [B, 16, h, w]);
    const v = await this.forwardDevice(lat, h, w, cond, tc, onBlock);
    lat.release();
    const o = await gpu.read(v);
    v.release();
    const vs = [];
    for (let bb = 0; bb < B; bb++) vs.push(o.slice(bb * per, (bb + 1) * per));
    return vs;
  }

  // forward on device tensors: lat [B, 16, h, w] -> velocities [B, 16, h, w] (a new tensor);
  // nothing is read back.
  async forwardDevice(lat, h, w, cond, tc, onBlock) {
    const gpu = this.gpu;
    const B = lat.shape[0];
    if (cond.B !== B) throw new Error(`forward: ${B} latents but ${cond.B} contexts`);
    if (lat.size !== B * 16 * h * w) throw new Error(`forward: latents of ${lat.size} values for B=${B} ${h}x${w}`);
    const Hp = h / 2, Wp = w / 2, L = Hp * Wp, M = B * L;
    const xin = gpu.empty([M, 68]);
    native.patchify(gpu.ctx, lat.buf, B, h, w, xin.buf);
    const x = ops.linear(gpu, xin, this.xEmbed);
    xin.release();
    const cs = this.ropeTable(Hp, Wp);

    for (let i = 0; i < this.blocks.length; i++) {
      const b = this.blocks[i];
      const m = tc.blocks[i];

      // self-attention: stacked QKV GEMM, then attention with q/k RMSNorm + RoPE fused.  With an
      // int8 / W4 stacked weight (LoRAs through its fused factors) and bf16 attention, the GEMM's
      // epilogue writes K (normed, rotated) and V^T straight into the attention's operand layout.
      let nf;
      let a;
      if (b.self.qkv && this.fuseQkv && this.precision === "bf16" && ops.qkvFusable(b.self.qkv, L, HEADS)) {
        nf = normFor(gpu, x, m.self, b.self.qkv);
        const f = ops.linearQkv(gpu, null, b.self.qkv, { B, L, H: HEADS, xq: nf.xq, xr: nf.xq.xr, kNorm: b.self.kn, cs,
          qNorm: b.self.qn, prepareQ: true });
        releaseNorm(nf);
        a = ops.attention(gpu, { qPrep: f.qPrep, kvPrep: f.kvPrep, B, Lq: L, Lk: L, H: HEADS, D: HD, ldq: D,
          precision: "bf16", oBf16: bf16Out(b.self.o, "bf16") });
        f.qPrep.release();
        f.kvPrep.release();
      } else {
        let qkv;
        if (b.self.qkv) {
          nf = normFor(gpu, x, m.self, b.self.qkv);
          qkv = project(gpu, nf, b.self.qkv, M, { name: "dit.self.qkv" });
          releaseNorm(nf);
        } else {
          qkv = projectParts(gpu, x, m.self, [b.self.q, b.self.k, b.self.v], M);
        }
        a = ops.attention(gpu, { q: qkv, k: qkv, v: qkv, B, Lq: L, Lk: L, H: HEADS, D: HD, ldq: 3 * D, ldk: 3 * D,
          ldv: 3 * D, qOff: 0, kOff: D, vOff: 2 * D, qNorm: b.self.qn, kNorm: b.self.kn, cs, precision: this.precision,
          oBf16: bf16Out(b.self.o, this.precision) });
        qkv.release();
      }
      outProject(gpu, a, b.self.o, M, x, m.self);
      a.release();

      // cross-attention against the per-prompt cached keys/values (q RMSNorm fused, no RoPE).  With
      // an int8 / W4 q projection (no LoRA) and bf16 attention, the GEMM's
      // epilogue writes Q as the attention's prepared operand (RMS-normed, scaled, bf16).
      nf = normFor(gpu, x, m.cross, b.cross.q);
      const kv = cond.kv[i];
      if (this.fuseQkv && cond.precision === "bf16" && ops.qFusable(b.cross.q, L, HEADS)) {
        const f = ops.linearQkv(gpu, null, b.cross.q, { B, L, H: HEADS, xq: nf.xq, xr: nf.xq.xr, qNorm: b.cross.qn,
          prepareQ: true });
        releaseNorm(nf);
        a = ops.attention(gpu, { qPrep: f.qPrep, kvPrep: kv.prep, B, Lq: L, Lk: cond.Lk, H: HEADS, D: HD, ldq: D,
          precision: "bf16", oBf16: bf16Out(b.cross.o, "bf16") });
        f.qPrep.release();
      } else {
        const q = project(gpu, nf, b.cross.q, M);
        releaseNorm(nf);
        a = ops.attention(gpu, { q, kvPrep: kv.prep, B, Lq: L, Lk: cond.Lk, H: HEADS, D: HD, ldq: D, qNorm: b.cross.qn,
          precision: cond.precision, oBf16: bf16Out(b.cross.o, cond.precision) });
        q.release();
      }
      outProject(gpu, a, b.cross.o, M, x, m.cross);
      a.release();

      // MLP.  With a quantized layer2 (and no LoRA on it that needs the fp32 GELU output), layer1
      // stores its pre-activation and the GELU runs in layer2's Hadamard + int8 pass, off the
      // GEMM epilogue; the int8 rows are the same.
      nf = normFor(gpu, x, m.mlp, b.l1);
      if (ops.needsRotation(b.l2) && !wantsXr(b.l2)) {
        const pre = project(gpu, nf, b.l1, M);
        releaseNorm(nf);
        const hq = ops.quantRows(gpu, pre, MLP, true, "gelu");
        pre.release();
        ops.linear(gpu, null, b.l2, { M, xq: hq, out: x, resid: true, gate: m.mlp, gOff: 2 * D });
        hq.release();
      } else {
        const hdn = project(gpu, nf, b.l1, M, { act: "gelu" });
        releaseNorm(nf);
        ops.linear(gpu, hdn, b.l2, { M, out: x, resid: true, gate: m.mlp, gOff: 2 * D });
        hdn.release();
      }

      gpu.flush();
      if (onBlock) await onBlock(i, x);
    }

    const n = ops.layernormMod(gpu, x, tc.final, 0, D, D, false);
    x.release();
    const out = ops.linear(gpu, n, this.finalLinear); // [M, 64] = (p1 p2 c)
    n.release();
    const v = gpu.empty([B, 16, h, w]);
    native.unpatchify(gpu.ctx, out.buf, B, h, w, v.buf); // dit.js:68-78 on the device
    out.release();
    return v;
  }
}

// forwardDevice recorded once into a HIP graph (anima_graph_*) and replayed: the same ~600
// kernels with the same arguments, submitted as one graph launch instead of one launch each.
// A replay reads `lat` and the graph's timeCond slot as they are when it runs and overwrites
// `v`.  Capture needs the RoPE table to be cached (and is cheapest when the pool already holds
// the forward's buffers): with `warm` it runs the forward once eagerly first; without, the caller
// has just run forwardDevice for the same shapes.  The attention scratch of the captured calls is
// the graph's own (sized for them), not the context's workspace.  Recording itself executes nothing.
export class ForwardGraph {
  constructor(dit, graph, lat, v, tc) {
    this.dit = dit;
    this.gpu = dit.gpu;
    this.graph = graph;
    this.lat = lat;
    this.v = v;
    this.tc = tc;
  }

  // lat: the [B, 16, h, w] input tensor (kept allocated by the caller while the graph lives);
  // tcLike: a timeCond result (its layout and initial values).
  static async capture(dit, lat, h, w, cond, tcLike, warm) {
    const gpu = dit.gpu;
    const tc = dit.timeCondSlot(tcLike);
    dit.copyTimeCond(tc, tcLike);
    if (warm !== false) (await dit.forwardDevice(lat, h, w, cond, tc)).release();
    native.graphBegin(gpu.ctx);
    let v = null, graph = 0;
    try {
      v = await dit.forwardDevice(lat, h, w, cond, tc);
    } finally {
      if (v) graph = native.graphEnd(gpu.ctx);
      else {
        try {
          native.graphDestroy(gpu.ctx, native.graphEnd(gpu.ctx));
        } catch (e) {
          // the capture was already invalid: graphEnd discarded it
        }
        tc.release();
      }
    }
    return new ForwardGraph(dit, graph, lat, v, tc);
  }

  // Replays the forward with the modulation vectors of timeCond result `tc` (copied into the
  // slot unless it is the slot); returns the velocities [B, 16, h, w] (owned by the graph).
  run(tc) {
    if (tc && tc !== this.tc) this.dit.copyTimeCond(this.tc, tc);
    native.graphLaunch(this.gpu.ctx, this.graph);
    return this.v;
  }

  release() {
    if (this.graph) native.graphDestroy(this.gpu.ctx, this.graph);
    this.graph = 0;
    if (this.v) this.v.release();
    this.v = null;
    if (this.tc) this.tc.release();
    this.tc = null;
  }
}

// ------------------------------------------------------------------ LLM adapter
// Maps the text encoder's hidden states and T5 token ids to the DiT's [512, 1024] context
// (app/models/dit.js:136-190; tools/reference.py:141-169): 6 blocks of RMSNorm -> self-attention
// over the T5 tokens, RMSNorm -> cross-attention to the text encoder's tokens (16 heads x 64,
// q/k RMSNorm, 1D RoPE theta 1e4 on both sides), RMSNorm -> GELU MLP (biased); then out_proj,
// RMSNorm, the per-token prompt weights, zero rows up to 512.
export const ADAPTER = { blocks: 6, dim: 1024, heads: 16, headDim: 64, mlp: 4096, theta: 1e4, ctxLen: 512 };

// Adapter weights in the reference's names (app/models/dit.js:13-22, 84-100).
export function loadAdapter(gpu, st) {
  const attn = (p) => ({
    q: st.linear(gpu, p + "q_proj."), k: st.linear(gpu, p + "k_proj."), v: st.linear(gpu, p + "v_proj."),
    o: st.linear(gpu, p + "o_proj."), qn: st.vector(gpu, p + "q_norm.weight"), kn: st.vector(gpu, p + "k_norm.weight"),
  });
  const A = { blocks: [] };
  for (let i = 0; i < ADAPTER.blocks; i++) {
    const p = `llm_adapter.blocks.${i}.`;
    A.blocks.push({
      nSelf: st.vector(gpu, p + "norm_self_attn.weight"), nCross: st.vector(gpu, p + "norm_cross_attn.weight"),
      nMlp: st.vector(gpu, p + "norm_mlp.weight"), self: attn(p + "self_attn."), cross: attn(p + "cross_attn."),
      mlp0: st.linear(gpu, p + "mlp.0."), mlp2: st.linear(gpu, p + "mlp.2."),
    });
  }
  A.outProj = st.linear(gpu, "llm_adapter.out_proj.");
  A.norm = st.vector(gpu, "llm_adapter.norm.weight");
  A.embedRows = (ids) => st.rows("llm_adapter.embed.weight", ids);
  return A;
}

// Seeded random-init adapter (bf16 linears, biases on the MLP and out_proj as in the checkpoint,
// an embedding table of `vocab` rows); opts: { blocks, vocab }.
export function syntheticAdapter(gpu, src, opts) {
  const o = opts || {};
  const D = ADAPTER.dim, F = ADAPTER.mlp, HD = ADAPTER.headDim;
  const lin = (name, N, K, gain, bias) => {
    const W = src.bf16Linear(gpu, name, N, K, gain);
    if (bias) W.bias = src.vector(gpu, name + ".bias", N, -0.02, 0.02);
    return W;
  };
  const attn = (p) => ({
    q: lin(p + "q", D, D, 1.0), k: lin(p + "k", D, D, 1.0), v: lin(p + "v", D, D, 1.0), o: lin(p + "o", D, D, 0.5),
    qn: src.vector(gpu, p + "qn", HD), kn: src.vector(gpu, p + "kn", HD),
  });
  const A = { blocks: [] };
  for (let i = 0; i < (o.blocks || ADAPTER.blocks); i++) {
    const p = `ad.${i}.`;
    A.blocks.push({
      nSelf: src.vector(gpu, p + "ns", D), nCross: src.vector(gpu, p + "nc", D), nMlp: src.vector(gpu, p + "nm", D),
      self: attn(p + "s."), cross: attn(p + "c."), mlp0: lin(p + "m0", F, D, 1.0, true), mlp2: lin(p + "m2", D, F, 0.5, true),
    });
  }
  A.outProj = lin("ad.out", D, D, 1.0, true);
  A.norm = src.vector(gpu, "ad.norm", D);
  const vocab = o.vocab || 1024;
  A.table = src.fill(gpu.empty([vocab * D]), "f32", "ad.embed", -1, 1);
  A.embedRows = async (ids) => {
    const all = await gpu.read(A.table);
    const out = new Float32Array(ids.length * D);
    ids.forEach((id, i) => out.set(all.subarray(id * D, (id + 1) * D), i * D));
    return out;
  };
  return A;
}

// hidden: Tensor [Ls, 1024] from the text encoder; t5Ids / t5Weights: arrays.  Returns the context
// Tensor [max(512, Lt), 1024] (app/models/dit.js:136-190).  precision: attention precision.
export async function adapt(gpu, A, hidden, t5Ids, t5Weights, precision) {
  const D = ADAPTER.dim, H = ADAPTER.heads, HD = ADAPTER.headDim;
  const Lt = t5Ids.length, Ls = hidden.shape[0];
  const x = gpu.fromArray(await A.embedRows(t5Ids), [Lt, D]);
  const csT = ropeTable(gpu, Lt, HD, ADAPTER.theta);
  const csS = ropeTable(gpu, Ls, HD, ADAPTER.theta);
  const attn = (w, xq, ctx, Lq, Lk, csQ, csK) => {
    const q = ops.linear(gpu, xq, w.q);
    const k = ops.linear(gpu, ctx, w.k);
    const v = ops.linear(gpu, ctx, w.v);
    const qn = ops.rmsnorm(gpu, q, w.qn, HD);
    const kn = ops.rmsnorm(gpu, k, w.kn, HD);
    q.release();
    k.release();
    ops.rope(gpu, qn, csQ, Lq, H, HD);
    ops.rope(gpu, kn, csK, Lk, H, HD);
    const a = ops.attention(gpu, { q: qn, k: kn, v, Lq, Lk, H, D: HD, ldq: D, ldk: D, ldv: D, precision });
    releaseAll([qn, kn, v]);
    ops.linear(gpu, a, w.o, { out: x, resid: true });
    a.release();
  };
  for (const b of A.blocks) {
    let n = ops.rmsnorm(gpu, x, b.nSelf, D);
    attn(b.self, n, n, Lt, Lt, csT, csT);
    n.release();
    n = ops.rmsnorm(gpu, x, b.nCross, D);
    attn(b.cross, n, hidden, Lt, Ls, csT, csS);
    n.release();
    n = ops.rmsnorm(gpu, x, b.nMlp, D);
    const h = ops.linear(gpu, n, b.mlp0, { act: "gelu" });
    n.release();
    ops.linear(gpu, h, b.mlp2, { out: x, resid: true });
    h.release();
  }
  releaseAll([csT, csS]);
  const o = ops.linear(gpu, x, A.outProj);
  x.release();
  const on = ops.rmsnorm(gpu, o, A.norm, D);
  o.release();
  // prompt weights and zero rows up to 512 (on the host, as the reference: tiny)
  const vals = await gpu.read(on);
  on.release();
  const ctx = new Float32Array(Math.max(ADAPTER.ctxLen, Lt) * D);
  for (let i = 0; i < Lt; i++) {
    const w = t5Weights ? t5Weights[i] : 1;
    for (let j = 0; j < D; j++) ctx[i * D + j] = vals[i * D + j] * w;
  }
  return gpu.fromArray(ctx, [ctx.length / D, D]);
}
