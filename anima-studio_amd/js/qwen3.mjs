// The Qwen3-0.6B text encoder of Anima (app/models/qwen3.js:1-79) on this build's ops: 28 layers
// of RMSNorm -> q/k/v linears -> per-head q/k RMSNorm -> 1D RoPE -> causal GQA attention (16 query
// heads over 8 kv heads, on the flash kernels) -> o linear (residual) -> RMSNorm -> gate/up
// linears -> SiLU(gate) * up -> down linear (residual); the final RMSNorm's output is the hidden
// state the DiT's context is built from.  Node-12 syntax only.

import * as ops from "./ops.mjs";
import { ropeTable } from "./common.mjs";
import { concatLinears } from "./weights.mjs";
import { native } from "./gpu.mjs";

function releaseGraph(gpu, g) {
  native.graphDestroy(gpu.ctx, g.graph);
  for (const t of [g.out, g.x, g.cs]) t.release();
}

// q, k and v of a layer stacked into one [(H + 2 KH) HD, D] linear (one GEMM per layer instead
// of three; the q/k RMSNorm and RoPE then run inside the attention's loads).  Formats that
// cannot be stacked (W4 parts with different codebooks) keep the three linears.
function stackQKV(gpu, l) {
  const qkv = concatLinears(gpu, [l.q, l.k, l.v]);
  if (!qkv) return;
  l.qkv = qkv;
  delete l.q;
  delete l.k;
  delete l.v;
}

export const QWEN3 = { layers: 28, hidden: 1024, heads: 16, kvHeads: 8, headDim: 128, mlp: 3072, theta: 1e6, vocab: 151936 };

export class Qwen3 {
  // Weights from a safetensors file in the reference's names (qwen3.js:8-31).
  static async load(gpu, st, onProgress) {
    const m = new Qwen3(gpu, QWEN3);
    m.layers = [];
    for (let i = 0; i < QWEN3.layers; i++) {
      const p = `model.layers.${i}.`;
      m.layers.push({
        ln1: st.vector(gpu, p + "input_layernorm.weight"),
        ln2: st.vector(gpu, p + "post_attention_layernorm.weight"),
        qn: st.vector(gpu, p + "self_attn.q_norm.weight"),
        kn: st.vector(gpu, p + "self_attn.k_norm.weight"),
        q: st.linear(gpu, p + "self_attn.q_proj."),
        k: st.linear(gpu, p + "self_attn.k_proj."),
        v: st.linear(gpu, p + "self_attn.v_proj."),
        o: st.linear(gpu, p + "self_attn.o_proj."),
        gate: st.linear(gpu, p + "mlp.gate_proj."),
        up: st.linear(gpu, p + "mlp.up_proj."),
        down: st.linear(gpu, p + "mlp.down_proj."),
      });
      stackQKV(gpu, m.layers[i]);
      if (onProgress) onProgress((i + 1) / QWEN3.layers);
    }
    m.norm = st.vector(gpu, "model.norm.weight");
    m.embedRows = (ids) => st.rows("model.embed_tokens.weight", ids);
    return m;
  }

  // Seeded random-init weights of the same architecture (bf16 linears, norm weights near 1, an
  // embedding table of `vocab` rows held on the host); opts: { layers, vocab }.
  static synthetic(gpu, src, opts) {
    const o = opts || {};
    const cfg = Object.assign({}, QWEN3, { layers: o.layers || QWEN3.layers, vocab: o.vocab || 4096 });
    const m = new Qwen3(gpu, cfg);
    const { hidden: D, heads: H, kvHeads: KH, headDim: HD, mlp: F } = cfg;
    m.layers = [];
    for (let i = 0; i < cfg.layers; i++) {
      // the checkpoint's module names (qwen3.js:8-31), so that LoRA files address these linears
      const p = `model.layers.${i}.`;
      m.layers.push({
        ln1: src.vector(gpu, p + "input_layernorm.weight", D), ln2: src.vector(gpu, p + "post_attention_layernorm.weight", D),
        qn: src.vector(gpu, p + "self_attn.q_norm.weight", HD), kn: src.vector(gpu, p + "self_attn.k_norm.weight", HD),
        q: src.bf16Linear(gpu, p + "self_attn.q_proj", H * HD, D, 1.0), k: src.bf16Linear(gpu, p + "self_attn.k_proj", KH * HD, D, 1.0),
        v: src.bf16Linear(gpu, p + "self_attn.v_proj", KH * HD, D, 1.0), o: src.bf16Linear(gpu, p + "self_attn.o_proj", D, H * HD, 0.5),
        gate: src.bf16Linear(gpu, p + "mlp.gate_proj", F, D, 1.0), up: src.bf16Linear(gpu, p + "mlp.up_proj", F, D, 1.0),
        down: src.bf16Linear(gpu, p + "mlp.down_proj", D, F, 0.5),
      });
      stackQKV(gpu, m.layers[i]);
    }
    m.norm = src.vector(gpu, "model.norm.weight", D);
    const table = gpu.empty([cfg.vocab * D]);
    src.fill(table, "f32", "model.embed_tokens.weight", -1, 1);
    m.table = table;
    m.embedRows = async (ids) => {
      const all = await gpu.read(table);
      const out = new Float32Array(ids.length * D);
      ids.forEach((id, i) => out.set(all.subarray(id * D, (id + 1) * D), i * D));
      return out;
    };
    return m;
  }

  constructor(gpu, cfg) {
    this.gpu = gpu;
    this.cfg = cfg;
    this.precision = "bf16"; // attention precision ("fp32": the fp32-MFMA kernel)
    this.graphs = true; // replay the layers from a recorded HIP graph (per token count and precision)
    this.graphCache = new Map();
  }

  // ids -> Tensor [L, 1024] (qwen3.js:38-78).  With this.graphs (the default) the 28 layers run as a
  // HIP graph recorded once per (token count, attention precision): the host only uploads the
  // embedding rows and replays it (the same kernels and arguments as the eager pass, so the same
  // result), which removes the per-kernel launch cost of ~280 short kernels.
  async encode(ids) {
    const gpu = this.gpu;
    const { hidden: D, headDim: HD } = this.cfg;
    const Lt = ids.length;
    const rows = await this.embedRows(ids);
    // LoRA side paths (attachLoras) run eagerly: a graph recorded before an attach would not hold them
    const lora = this.layers.some((l) => ["qkv", "q", "k", "v", "o", "gate", "up", "down"].some((k) => l[k] && l[k].lora && l[k].lora.length));
    if (!this.graphs || lora) {
      const x = gpu.fromArray(rows, [Lt, D]);
      const cs = ropeTable(gpu, Lt, HD, this.cfg.theta);
      const out = this.layersDevice(x, cs, Lt);
      cs.release();
      x.release();
      return out;
    }
    const key = `${Lt}:${this.precision}`;
    let g = this.graphCache.get(key);
    if (!g) {
      g = this.recordGraph(rows, Lt);
      if (this.graphCache.size >= 4) {
        const [k0, g0] = this.graphCache.entries().next().value;
        this.graphCache.delete(k0);
        releaseGraph(gpu, g0);
      }
    } else {
      this.graphCache.delete(key);  // most recently used last
    }
    this.graphCache.set(key, g);
    gpu.write(g.x, rows);
    native.graphLaunch(gpu.ctx, g.graph);
    const out = gpu.empty([Lt, D]);
    gpu.copy(out, g.out, Lt * D * 4);
    return out;
  }

  // The fixed residual-stream buffer, RoPE table and output of one token count, and the graph of
  // the layers over them (recorded after one eager pass, so the pool already holds its buffers).
  recordGraph(rows, Lt) {
    const gpu = this.gpu;
    const { hidden: D, headDim: HD } = this.cfg;
    const x = gpu.fromArray(rows, [Lt, D]);
    const cs = ropeTable(gpu, Lt, HD, this.cfg.theta);
    this.layersDevice(x, cs, Lt).release();
    native.graphBegin(gpu.ctx);
    let out = null, graph = 0;
    try {
      out = this.layersDevice(x, cs, Lt);
    } finally {
      if (out) graph = native.graphEnd(gpu.ctx);
      else {
        try {
          native.graphDestroy(gpu.ctx, native.graphEnd(gpu.ctx));
        } catch (e) {
          // the capture was already invalid: graphEnd discarded it
        }
        x.release();
        cs.release();
      }
    }
    return { x, cs, out, graph };
  }

  // The decoder layers and the final RMSNorm on the residual stream x [Lt, D] (updated in place);
  // returns the normed hidden states (a new tensor).
  layersDevice(x, cs, Lt) {
    const gpu = this.gpu;
    const { hidden: D, heads: H, kvHeads: KH, headDim: HD } = this.cfg;
    for (const l of this.layers) {
      const h = ops.rmsnorm(gpu, x, l.ln1, D);
      const hr = ops.needsRotation(l.qkv || l.q) ? ops.rotate(gpu, h) : null;
      let a;
      if (l.qkv) {
        // one GEMM for q, k and v; their per-head RMSNorm and RoPE run in the attention's loads
        const qkv = ops.linear(gpu, h, l.qkv, { xr: hr });
        const ld = (H + 2 * KH) * HD;
        a = ops.attention(gpu, { q: qkv, k: qkv, v: qkv, Lq: Lt, Lk: Lt, H, D: HD, ldq: ld, ldk: ld, ldv: ld, qOff: 0,
          kOff: H * HD, vOff: (H + KH) * HD, group: H / KH, causal: true, qNorm: l.qn, kNorm: l.kn, cs,
          precision: this.precision });
        qkv.release();
      } else {
        const q = ops.linear(gpu, h, l.q, { xr: hr });
        const k = ops.linear(gpu, h, l.k, { xr: hr });
        const v = ops.linear(gpu, h, l.v, { xr: hr });
        const qn = ops.rmsnorm(gpu, q, l.qn, HD);
        const kn = ops.rmsnorm(gpu, k, l.kn, HD);
        q.release();
        k.release();
        ops.rope(gpu, qn, cs, Lt, H, HD);
        ops.rope(gpu, kn, cs, Lt, KH, HD);
        a = ops.attention(gpu, { q: qn, k: kn, v, Lq: Lt, Lk: Lt, H, D: HD, ldq: H * HD, ldk: KH * HD, ldv: KH * HD,
          group: H / KH, causal: true, precision: this.precision });
        qn.release();
        kn.release();
        v.release();
      }
      if (hr) hr.release();
      h.release();
      ops.linear(gpu, a, l.o, { out: x, resid: true });
      a.release();
      const h2 = ops.rmsnorm(gpu, x, l.ln2, D);
      const h2r = ops.needsRotation(l.gate) ? ops.rotate(gpu, h2) : null;
      const g = ops.linear(gpu, h2, l.gate, { xr: h2r });
      const u = ops.linear(gpu, h2, l.up, { xr: h2r });
      if (h2r) h2r.release();
      h2.release();
      const gu = ops.elementwise(gpu, "silu_mul", g, u);
      g.release();
      u.release();
      ops.linear(gpu, gu, l.down, { out: x, resid: true });
      gu.release();
    }
    return ops.rmsnorm(gpu, x, this.norm, D);
  }

  release() {
    const rel = (t) => {
      if (!t) return;
      if (t.buf && t.buf.release) t.buf.release();
      else if (t.release) t.release();
      for (const f of ["scale", "srel", "codebook", "bias"]) if (t[f] && t[f].release) t[f].release();
    };
    for (const g of this.graphCache.values()) releaseGraph(this.gpu, g);
    this.graphCache.clear();
    for (const l of this.layers || []) for (const key of Object.keys(l)) rel(l[key]);
    rel(this.norm);
    rel(this.table);
    this.layers = [];
  }
}
