// Runs one op case through the JS op layer (ops.mjs -> N-API -> libanima.so) for the parity
// tests: reads a JSON spec whose inputs are raw little-endian files, writes the outputs the same
// way.  node run_case.mjs case.json
//
// Cases:
//   attention  fused self-attention from a QKV file with q/k RMSNorm and the JS-built RoPE table
//   qknr       ops.qkNormRope in place
//   linear     ops.linear (i8 / w4 / bf16 weight files), with xr / resid / gate options
//   lnmod      ops.layernormMod (rotate) and ops.layernormModQ
//   dit        AnimaDiT.load(safetensors) -> timeCond -> prepareContext -> forward
//   lora       ops.linear with LoRA entries given as files (A in the input's basis), optional act,
//              stacked A matrices and a rotated-only input
//   loraq      ops.linear on int8 rows (quantRows) with fused LoRA factors: the A product over the
//              int8 rows (the default LoRA input) and over the fp32 rotated rows (setLoraInput)
//   lorafile   loadLora(safetensors) onto a 1-block synthetic DiT, then the block's stacked qkv
//              and mlp.layer2 linears with and without the attached LoRA
//   lorate     loadLora(safetensors) onto a 2-layer synthetic text encoder (text-encoder names):
//              layer 1's q_proj and mlp.down_proj with and without the LoRA, and the encoding
//   loramod    timeCond of a 1-block synthetic DiT with LoRAs on the adaLN modulation linears,
//              on the fused (grouped GEMV) and the per-linear modulation paths
//   generate   LatentPipeline.generate (device loop) and generateHost (the reference's host loop)
//              on a synthetic DiT, per sampler / scheduler / cfg
//   graph      ForwardGraph replays against eager forwardDevice on a synthetic DiT: one replay per
//              sigma, a new input latent and an eager forward before each
//   qwen3      Qwen3.encode of a synthetic text encoder (both attention precisions) and its
//              weights, for the oracle's restatement of qwen3.js
//   adapter    the LLM adapter (dit.mjs adapt) on a synthetic adapter, both attention precisions,
//              and its weights
//   chain      prompt tokens -> Qwen3.encode -> adapt -> prepareContext -> forward (synthetic
//              weights, cond + uncond prompts), the velocities
//   synthdit   a seeded synthetic DiT (any depth) on given latents and contexts: velocities and the
//              residual stream after block 0, for the oracle's restatement of the same weights
//   loradit    a seeded synthetic DiT with seeded LoRAs on every block linear: the forward without
//              LoRAs, with them on the int8 rows (default) and on the fp32 rows (setLoraInput)
//   fullstep   the full-size CFG step of a synthetic DiT: eager, with equal contexts, and replayed
//              from a HIP graph
//   vae        VAEDecoder.decode of a seeded synthetic decoder: raw output, RGBA bytes, stages
//   pipeline   LatentPipeline.generate with a VAE: progress events, the image, a cancelled run

import fs from "fs";
import { GPU, native } from "../../anima-studio_amd/js/gpu.mjs";
import * as ops from "../../anima-studio_amd/js/ops.mjs";
import { ditRopeTable } from "../../anima-studio_amd/js/common.mjs";
import { SafeTensors } from "../../anima-studio_amd/js/weights.mjs";
import { AnimaDiT, ForwardGraph, syntheticAdapter, adapt } from "../../anima-studio_amd/js/dit.mjs";
import { SyntheticWeights } from "../../anima-studio_amd/js/weights.mjs";
import { linearRegistry, loadLora, attachLoras, destroyLora, rotatedA } from "../../anima-studio_amd/js/lora.mjs";
import { LatentPipeline } from "../../anima-studio_amd/js/pipeline.mjs";
import { TorchGenerator } from "../../anima-studio_amd/js/rng.mjs";
import { Qwen3 } from "../../anima-studio_amd/js/qwen3.mjs";
import { VAEDecoder } from "../../anima-studio_amd/js/vae.mjs";

const ARR = { f32: Float32Array, i8: Int8Array, u8: Uint8Array, u16: Uint16Array, i32: Int32Array };

function load(path, dtype) {
  const b = fs.readFileSync(path);
  const ab = b.buffer.slice(b.byteOffset, b.byteOffset + b.length);
  return new ARR[dtype || "f32"](ab);
}

function save(path, arr) {
  fs.writeFileSync(path, Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));
}

function weightFromFiles(gpu, w) {
  const W = { kind: w.kind, N: w.N, K: w.K, name: "case" };
  if (w.kind === "i8") {
    W.buf = gpu.upload(load(w.w, "i8"));
    W.scale = gpu.upload(load(w.scale));
  } else if (w.kind === "w4") {
    W.buf = gpu.upload(load(w.w, "u8"));
    W.srel = gpu.upload(load(w.srel, "u8"));
    W.scale = gpu.upload(load(w.scale));
    W.codebookData = load(w.codebook);
    W.codebook = gpu.upload(W.codebookData);
  } else {
    W.buf = gpu.upload(load(w.w, "u16"));
  }
  if (w.bias) W.bias = gpu.upload(load(w.bias));
  return W;
}

async function main() {
  const spec = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  const gpu = await GPU.create({});
  const c = spec;
  if (c.case === "attention") {
    const L = c.Hp * c.Wp, H = c.H, D = 128;
    const qkv = gpu.fromArray(load(c.qkv), [c.B * L, 3 * H * D]);
    const qn = gpu.upload(load(c.qn)), kn = gpu.upload(load(c.kn));
    const cs = ditRopeTable(gpu, c.Hp, c.Wp);
    const o = ops.attention(gpu, { q: qkv, k: qkv, v: qkv, B: c.B, Lq: L, Lk: L, H, D, ldq: 3 * H * D, ldk: 3 * H * D,
      ldv: 3 * H * D, qOff: 0, kOff: H * D, vOff: 2 * H * D, qNorm: qn, kNorm: kn, cs, precision: c.precision });
    save(c.out, await gpu.read(o));
    save(c.out + ".cs", await gpu.read(cs));
  } else if (c.case === "qknr") {
    const L = c.Hp * c.Wp, H = c.H, D = 128;
    const qkv = gpu.fromArray(load(c.qkv), [L, 3 * H * D]);
    const cs = ditRopeTable(gpu, c.Hp, c.Wp);
    ops.qkNormRope(gpu, qkv, gpu.upload(load(c.qn)), gpu.upload(load(c.kn)), cs, L, H, D);
    save(c.out, await gpu.read(qkv));
  } else if (c.case === "linear") {
    const W = weightFromFiles(gpu, c.W);
    const x = gpu.fromArray(load(c.x), [c.M, W.K]);
    const opts = { act: c.act || "none" };
    if (c.xr) opts.xr = x;
    if (c.resid) {
      opts.out = gpu.fromArray(load(c.resid), [c.M, W.N]);
      opts.resid = true;
      if (c.gate) {
        opts.gate = gpu.upload(load(c.gate));
        opts.gOff = c.gOff;
      }
    }
    const y = ops.linear(gpu, x, W, opts);
    save(c.out, await gpu.read(y));
  } else if (c.case === "lora") {
    const W = weightFromFiles(gpu, c.W);
    const x = gpu.fromArray(load(c.x), [c.M, W.K]);
    const base = ops.linear(gpu, x, W, { act: c.act });
    save(c.out + ".base", await gpu.read(base));
    W.lora = c.lora.map((e) => {
      const A = gpu.upload(load(e.A));
      const Ar = ops.needsRotation(W) ? rotatedA(gpu, A, e.r * W.K) : null;
      return { A, Ar, B: gpu.upload(load(e.B)), r: e.r, scale: e.scale, off: e.off, n: e.n };
    });
    if (c.stack) ops.stackLora(gpu, W);
    // rotated: the caller holds only the rotated input (the fused LayerNorm path)
    const y = ops.linear(gpu, c.rotated ? null : x, W, { act: c.act, M: c.M, xr: c.rotated ? ops.rotate(gpu, x) : undefined });
    save(c.out, await gpu.read(y));
    ops.releaseLoraStack(W);
  } else if (c.case === "loraq") {
    const W = weightFromFiles(gpu, c.W);
    const x = gpu.fromArray(load(c.x), [c.M, W.K]);
    const xq = ops.quantRows(gpu, x, W.K, true);
    save(c.out + ".q", await gpu.read(xq.q));
    save(c.out + ".s", await gpu.read(xq.s));
    save(c.out + ".base", await gpu.read(ops.linear(gpu, null, W, { act: c.act, M: c.M, xq })));
    W.lora = c.lora.map((e) => {
      const A = gpu.upload(load(e.A));
      return { A, Ar: rotatedA(gpu, A, e.r * W.K), B: gpu.upload(load(e.B)), r: e.r, scale: e.scale, off: e.off, n: e.n };
    });
    ops.fuseLora(gpu, W);
    if (!ops.loraReadsInt8(W)) throw new Error("the fused LoRA factors should read the int8 rows");
    save(c.out, await gpu.read(ops.linear(gpu, null, W, { act: c.act, M: c.M, xq })));
    ops.setLoraInput("fp32");
    const xr = ops.rotate(gpu, x);
    save(c.out + ".fp32", await gpu.read(ops.linear(gpu, null, W, { act: c.act, M: c.M, xq, xr })));
    ops.setLoraInput("int8");
    ops.releaseLoraFused(W);
  } else if (c.case === "lorafile") {
    const src = new SyntheticWeights(gpu, 7, { mode: c.mode, blocks: 1 });
    const dit = AnimaDiT.synthetic(gpu, src);
    const regs = { dit: linearRegistry(dit), te: null };
    const L = loadLora(gpu, c.lora, regs);
    const x = gpu.fromArray(load(c.x), [c.M, 2048]);
    const h = gpu.fromArray(load(c.h), [c.M, 8192]);
    const b = dit.blocks[0];
    save(c.out + ".qkv.base", await gpu.read(ops.linear(gpu, x, b.self.qkv, {})));
    save(c.out + ".l2.base", await gpu.read(ops.linear(gpu, h, b.l2, {})));
    attachLoras(regs, [{ lora: L, strength: c.strength }]);
    save(c.out + ".qkv", await gpu.read(ops.linear(gpu, x, b.self.qkv, {})));
    save(c.out + ".l2", await gpu.read(ops.linear(gpu, h, b.l2, {})));
    const entries = [b.self.qkv, b.l2].map((W) => W.lora.map((e) => ({ r: e.r, scale: e.scale, off: e.off, n: e.n })));
    console.log(JSON.stringify({ matched: L.matched, total: L.total, unsupported: L.unsupported, skipped: L.skipped, entries }));
    attachLoras(regs, []);
    destroyLora(L);
  } else if (c.case === "lorate") {
    const te = Qwen3.synthetic(gpu, new SyntheticWeights(gpu, 17), { layers: 2, vocab: 97 });
    const regs = { dit: null, te: linearRegistry(te) };
    const L = loadLora(gpu, c.lora, regs);
    const x = gpu.fromArray(load(c.x), [c.M, 1024]);
    const h = gpu.fromArray(load(c.h), [c.M, 3072]);
    const l = te.layers[1];
    const ids = [3, 14, 15, 92, 65, 35];
    const e0 = await te.encode(ids);
    save(c.out + ".enc.base", await gpu.read(e0));
    e0.release();
    // q_proj: its own linear, or the first H*HD columns of the stacked q/k/v linear
    const Wq = l.qkv || l.q;
    const nq = te.cfg.heads * te.cfg.headDim;
    const qCols = async (y) => {
      const all = await gpu.read(y);
      const out = new Float32Array(c.M * nq);
      for (let r = 0; r < c.M; r++) out.set(all.subarray(r * Wq.N, r * Wq.N + nq), r * nq);
      return out;
    };
    save(c.out + ".q.base", await qCols(ops.linear(gpu, x, Wq, {})));
    save(c.out + ".down.base", await gpu.read(ops.linear(gpu, h, l.down, {})));
    attachLoras(regs, [{ lora: L, strength: c.strength }]);
    save(c.out + ".q", await qCols(ops.linear(gpu, x, Wq, {})));
    save(c.out + ".down", await gpu.read(ops.linear(gpu, h, l.down, {})));
    const e1 = await te.encode(ids);
    save(c.out + ".enc", await gpu.read(e1));
    e1.release();
    const entries = [Wq, l.down].map((W) => W.lora.map((e) => ({ r: e.r, scale: e.scale, off: e.off, n: e.n })));
    console.log(JSON.stringify({ matched: L.matched, total: L.total, unsupported: L.unsupported, skipped: L.skipped, entries }));
    attachLoras(regs, []);
    destroyLora(L);
    te.release();
  } else if (c.case === "loramod") {
    const mods = async (tc) => {
      const parts = [tc.blocks[0].self, tc.blocks[0].cross, tc.blocks[0].mlp, tc.final];
      const arrs = [];
      for (const t of parts) arrs.push(await gpu.read(t));
      const out = new Float32Array(arrs.reduce((a, x) => a + x.length, 0));
      let o = 0;
      for (const x of arrs) { out.set(x, o); o += x.length; }
      return out;
    };
    const info = {};
    for (const fuse of [true, false]) {
      const tag = fuse ? "fused" : "plain";
      const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, 7, { mode: c.mode, blocks: 1 }), { fuse });
      const regs = { dit: linearRegistry(dit), te: null };
      const tc0 = dit.timeCond(c.sigma);
      save(`${c.out}.${tag}.base`, await mods(tc0));
      tc0.release();
      const L = loadLora(gpu, c.lora, regs);
      attachLoras(regs, [{ lora: L, strength: c.strength }]);
      const tc = dit.timeCond(c.sigma);
      save(`${c.out}.${tag}`, await mods(tc));
      tc.release();
      info[tag] = { matched: L.matched, skipped: L.skipped };
      attachLoras(regs, []);
      destroyLora(L);
    }
    console.log(JSON.stringify(info));
  } else if (c.case === "generate") {
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, 5, { mode: c.mode, blocks: c.blocks || 1 }));
    const pipe = new LatentPipeline(gpu, dit);
    const runs = {};
    for (const run of c.runs) {
      const B = run.cfg !== 1 ? 2 : 1;
      const ctxs = [];
      for (let b = 0; b < B; b++) ctxs.push(gpu.fromArray(new TorchGenerator(100 + b).randn(c.Lk * 1024), [c.Lk, 1024]));
      const cond = dit.prepareContext(ctxs);
      const opts = Object.assign({ cond, width: c.size, height: c.size }, run);
      const dev = await pipe.generate(opts);
      const host = await pipe.generateHost(opts);
      save(`${c.out}.${run.key}.dev`, dev.latent);
      save(`${c.out}.${run.key}.host`, host.latent);
      runs[run.key] = { steps: dev.sigmas.length - 1 };
      cond.release();
    }
    console.log(JSON.stringify({ runs, stats: pipe.stats }));
    pipe.clearTimeCache();
  } else if (c.case === "pipeline") {
    // LatentPipeline.generate with a VAE: progress events, the decoded image, and cancellation
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, 5, { mode: "int8", blocks: c.blocks }));
    const vae = VAEDecoder.synthetic(gpu, new SyntheticWeights(gpu, 21));
    const pipe = new LatentPipeline(gpu, dit, { vae });
    const ctxs = [0, 1].map((b) => gpu.fromArray(new TorchGenerator(100 + b).randn(c.Lk * 1024), [c.Lk, 1024]));
    const cond = dit.prepareContext(ctxs);
    const events = [];
    const opts = { cond, width: c.size, height: c.size, steps: c.steps, sampler: "euler", cfg: 3,
      onProgress: (e) => events.push(e) };
    const r = await pipe.generate(opts);
    save(c.out + ".latent", r.latent);
    save(c.out + ".img", r.image.data);
    // cancelled after the first progress event: the generation throws an AbortError
    const signal = { aborted: false };
    let cancel = null;
    try {
      await pipe.generate(Object.assign({}, opts, { signal, onProgress: () => { signal.aborted = true; } }));
    } catch (e) {
      cancel = { name: e.name, message: e.message };
    }
    console.log(JSON.stringify({ pipeline: { events, image: [r.image.width, r.image.height], cancel,
      timings: r.timings, pool: gpu.pool.allocated } }));
    cond.release();
    pipe.clearTimeCache();
  } else if (c.case === "graph") {
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, 9, { mode: c.mode, blocks: c.blocks }));
    const ctxs = [0, 1].map((b) => gpu.fromArray(new TorchGenerator(200 + b).randn(c.Lk * 1024), [c.Lk, 1024]));
    const cond = dit.prepareContext(ctxs);
    const h = c.size / 8, w = c.size / 8, n = 2 * 16 * h * w;
    const lat = gpu.empty([2, 16, h, w]);
    const tcs = c.sigmas.map((sg) => dit.timeCond(sg));
    gpu.write(lat, new TorchGenerator(300).randn(n));
    const fg = await ForwardGraph.capture(dit, lat, h, w, cond, tcs[0]);
    const diffs = [];
    for (let r = 0; r < tcs.length; r++) {
      gpu.write(lat, new TorchGenerator(400 + r).randn(n));
      const ev = await dit.forwardDevice(lat, h, w, cond, tcs[r]);
      const e = await gpu.read(ev);
      ev.release();
      const g = await gpu.read(fg.run(tcs[r]));
      let nd = 0;
      for (let i = 0; i < n; i++) if (e[i] !== g[i]) nd++;
      diffs.push(nd);
      save(`${c.out}.eager${r}`, e);
      save(`${c.out}.graph${r}`, g);
    }
    fg.release();
    for (const tc of tcs) tc.release();
    lat.release();
    cond.release();
    console.log(JSON.stringify({ graph: { diffs, n } }));
  } else if (c.case === "limits") {
    console.log(JSON.stringify({ limits: gpu.limits, maxBinding: gpu.maxBinding, info: gpu.info }));
  } else if (c.case === "leak") {
    // tensors dropped without release(): their finalizers return the buffers (run with --expose-gc)
    const bytes = c.mb * 1024 * 1024;
    const f0 = native.finalized();
    for (let i = 0; i < c.n; i++) {
      const t = gpu.empty([bytes / 4]);
      ops.zero(gpu, t);
      global.gc();
      await new Promise((r) => setImmediate(r));
    }
    global.gc();
    await new Promise((r) => setImmediate(r));
    const kept = gpu.empty([16]);
    kept.release();
    kept.release(); // a second release is a no-op
    const peak = gpu.pool.peak;
    console.log(JSON.stringify({ leak: { n: c.n, bytes, finalized: native.finalized() - f0, peak,
      released_twice_ok: kept.buf === 0 } }));
  } else if (c.case === "teardown") {
    // the process returns normally with tensors that were never released: some already collected
    // (their finalizers ran), some unreachable but not yet collected, some still referenced, and
    // the context left open; Node's environment teardown must not crash on them
    const kept = [];
    for (let i = 0; i < c.n; i++) {
      const t = gpu.empty([1024 * (i + 1)]);
      ops.zero(gpu, t);
      if (i % 3 === 0) kept.push(t);
      if (i === c.n >> 1 && global.gc) {
        global.gc();
        await new Promise((r) => setImmediate(r));
      }
    }
    globalThis.__kept = kept;
    await gpu.sync();
    console.log(JSON.stringify({ teardown: { n: c.n, kept: kept.length, finalized: native.finalized() } }));
    return; // no destroy(), no release(), no process.exit()
  } else if (c.case === "vae") {
    // the VAE decoder on seeded synthetic weights: raw output, RGBA image, progress stages
    const vae = VAEDecoder.synthetic(gpu, new SyntheticWeights(gpu, c.seed));
    vae.precision = c.precision || "fp32";
    vae.keepRaw = true;
    const stages = [];
    const r = await vae.decode(load(c.latent), c.h, c.w, (f) => stages.push(f));
    save(c.out + ".raw", r.raw);
    save(c.out + ".img", r.data);
    console.log(JSON.stringify({ vae: { width: r.width, height: r.height, stages } }));
  } else if (c.case === "synthdit") {
    // a seeded synthetic DiT (the weights the oracle restates by name) on given latents / contexts
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, c.seed, { mode: c.mode, blocks: c.blocks }));
    // unpackW4: W4 weights converted to their int8 grids at load first
    if (c.unpackW4) console.log(JSON.stringify({ unpacked: dit.unpackW4() }));
    const tc = dit.timeCond(c.sigma);
    const cond = dit.prepareContext(c.ctx.map((p) => gpu.fromArray(load(p), [c.Lk, 1024])));
    const blockOut = [];
    const v = await dit.forward(c.latents.map((p) => load(p)), c.h, c.w, cond, tc, async (i, x) => {
      if (i === 0) blockOut.push(await gpu.read(x));
    });
    v.forEach((vb, b) => save(c.out + "." + b, vb));
    save(c.out + ".block0", blockOut[0]);
    tc.release();
    cond.release();
  } else if (c.case === "loradit") {
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, c.seed, { mode: c.mode, blocks: c.blocks }));
    const regs = { dit: linearRegistry(dit), te: null };
    const lat = c.latents.map((p) => load(p));
    const forward = async (name) => {
      const tc = dit.timeCond(c.sigma);
      const cond = dit.prepareContext(c.ctx.map((p) => gpu.fromArray(load(p), [c.Lk, 1024])));
      const v = await dit.forward(lat, c.h, c.w, cond, tc);
      v.forEach((vb, b) => save(`${c.out}.${name}.${b}`, vb));
      tc.release();
      cond.release();
    };
    await forward("base");
    const modules = [], bufs = [];
    let seed = 700;
    for (const [name, t] of regs.dit) {
      if (!name.startsWith("blocks_")) continue;
      const A = gpu.empty([c.rank * t.W.K]), B = gpu.empty([t.n * c.rank]);
      native.fillRandom(gpu.ctx, A.buf, A.size, 4, seed++, 0.02, 0.0);
      native.fillRandom(gpu.ctx, B.buf, B.size, 4, seed++, 0.02, 0.0);
      const Ar = ops.needsRotation(t.W) ? rotatedA(gpu, A, A.size) : null;
      bufs.push(A, B, Ar);
      modules.push({ target: t, A, Ar, B, r: c.rank, alphaScale: 1 });
    }
    attachLoras(regs, [{ lora: { modules }, strength: 1 }]);
    const int8 = [...regs.dit.values()].filter(({ W }) => ops.loraReadsInt8(W)).length;
    await forward("int8");
    ops.setLoraInput("fp32");
    await forward("fp32");
    ops.setLoraInput("int8");
    attachLoras(regs, []);
    for (const t of bufs) if (t) t.release();
    console.log(JSON.stringify({ loradit: { modules: modules.length, int8 } }));
  } else if (c.case === "fullstep") {
    // the full-size CFG step: one latent in both batch halves (as LatentPipeline.generate feeds
    // it), the cond and uncond contexts; then the same step with the uncond context equal to the
    // cond one, and the step replayed from a HIP graph
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, c.seed, { mode: c.mode, blocks: c.blocks }));
    const h = c.size / 8, w = c.size / 8, n = 16 * h * w;
    const ctxA = [0, 1].map((b) => new TorchGenerator(200 + b).randn(c.Lk * 1024));
    const lat = gpu.empty([2, 16, h, w]);
    const x = new TorchGenerator(300).randn(n);
    gpu.write(lat, x);
    gpu.write(lat, x, n * 4);
    const tc = dit.timeCond(c.sigma);
    const run = async (ctxs) => {
      const cond = dit.prepareContext(ctxs.map((a) => gpu.fromArray(a, [c.Lk, 1024])));
      gpu.timerStart();
      const v = await dit.forwardDevice(lat, h, w, cond, tc);
      const ms = gpu.timerStop();
      const out = await gpu.read(v);
      v.release();
      return { cond, out, ms };
    };
    const a = await run(ctxA);
    const same = await run([ctxA[0], ctxA[0]]);
    same.cond.release();
    const fg = await ForwardGraph.capture(dit, lat, h, w, a.cond, tc, false);
    const g = await gpu.read(fg.run(tc));
    fg.release();
    a.cond.release();
    tc.release();
    lat.release();
    save(c.out + ".eager", a.out);
    save(c.out + ".same", same.out);
    save(c.out + ".graph", g);
    console.log(JSON.stringify({ fullstep: { n, ms: a.ms } }));
  } else if (c.case === "qwen3") {
    const te = Qwen3.synthetic(gpu, new SyntheticWeights(gpu, 17), { layers: c.layers, vocab: c.vocab });
    for (const prec of ["fp32", "bf16"]) {
      te.precision = prec;
      // graph replays (recorded on the first call, replayed on the second) and the eager pass
      te.graphs = true;
      for (const tag of ["", ".replay"]) {
        const y = await te.encode(c.ids);
        save(`${c.out}.${prec}${tag}`, await gpu.read(y));
        y.release();
      }
      te.graphs = false;
      const ye = await te.encode(c.ids);
      save(`${c.out}.${prec}.eager`, await gpu.read(ye));
      ye.release();
      te.graphs = true;
    }
    // a weight object holds its Tensor in .buf; a Tensor's .buf is its device address
    const dump = async (name, t) => save(`${c.out}.w.${name}`, await gpu.read(typeof t.buf === "object" ? t.buf : t));
    for (let i = 0; i < te.layers.length; i++) {
      const l = te.layers[i];
      for (const k of ["ln1", "ln2", "qn", "kn", "o", "gate", "up", "down"]) await dump(`${i}.${k}`, l[k]);
      if (l.qkv) {
        // q, k and v are row blocks of the stacked [(H + 2 KH) HD, D] weight
        const all = await gpu.read(l.qkv.buf);
        const K = l.qkv.K, nq = te.cfg.heads * te.cfg.headDim, nk = te.cfg.kvHeads * te.cfg.headDim;
        save(`${c.out}.w.${i}.q`, all.subarray(0, nq * K));
        save(`${c.out}.w.${i}.k`, all.subarray(nq * K, (nq + nk) * K));
        save(`${c.out}.w.${i}.v`, all.subarray((nq + nk) * K, (nq + 2 * nk) * K));
      } else {
        for (const k of ["q", "k", "v"]) await dump(`${i}.${k}`, l[k]);
      }
    }
    await dump("norm", te.norm);
    await dump("embed", te.table);
    te.release();
  } else if (c.case === "adapter") {
    const A = syntheticAdapter(gpu, new SyntheticWeights(gpu, 23), { blocks: c.blocks, vocab: c.vocab });
    const hidden = gpu.fromArray(new TorchGenerator(24).randn(c.Ls * 1024), [c.Ls, 1024]);
    for (const prec of ["fp32", "bf16"]) {
      const y = await adapt(gpu, A, hidden, c.ids, c.weights, prec);
      save(`${c.out}.${prec}`, await gpu.read(y));
      y.release();
    }
    save(`${c.out}.hidden`, await gpu.read(hidden));
    const dump = async (name, t) => save(`${c.out}.w.${name}`, await gpu.read(typeof t.buf === "object" ? t.buf : t));
    for (let i = 0; i < A.blocks.length; i++) {
      const b = A.blocks[i];
      for (const k of ["nSelf", "nCross", "nMlp"]) await dump(`${i}.${k}`, b[k]);
      for (const a of ["self", "cross"]) for (const k of ["q", "k", "v", "o", "qn", "kn"]) await dump(`${i}.${a}.${k}`, b[a][k]);
      for (const k of ["mlp0", "mlp2"]) {
        await dump(`${i}.${k}`, b[k]);
        await dump(`${i}.${k}.bias`, b[k].bias);
      }
    }
    await dump("out", A.outProj);
    await dump("out.bias", A.outProj.bias);
    await dump("norm", A.norm);
    await dump("embed", A.table);
  } else if (c.case === "chain") {
    const te = Qwen3.synthetic(gpu, new SyntheticWeights(gpu, 31), { layers: 2, vocab: 97 });
    const A = syntheticAdapter(gpu, new SyntheticWeights(gpu, 32), { blocks: 2, vocab: 64 });
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, 33, { mode: "int8", blocks: 1 }));
    const ctxs = [];
    for (const p of c.prompts) {
      const hidden = await te.encode(p.qwen);
      ctxs.push(await adapt(gpu, A, hidden, p.t5, p.weights));
      hidden.release();
    }
    const cond = dit.prepareContext(ctxs);
    const tc = dit.timeCond(0.7);
    const hw = c.size / 8, per = 16 * hw * hw;
    const lat = [0, 1].map((b) => new TorchGenerator(40 + b).randn(per));
    const v = await dit.forward(lat, hw, hw, cond, tc);
    v.forEach((vb, b) => save(`${c.out}.${b}`, vb));
    tc.release();
    cond.release();
    te.release();
  } else if (c.case === "encode") {
    // LatentPipeline.encode: per-prompt conditioning cache with keep-list eviction; stacked cached
    // conditionings give the same velocities as prepareContext over both contexts at once
    const te = Qwen3.synthetic(gpu, new SyntheticWeights(gpu, 31), { layers: 2, vocab: 97 });
    const A = syntheticAdapter(gpu, new SyntheticWeights(gpu, 32), { blocks: 2, vocab: 64 });
    const dit = AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, 33, { mode: "int8", blocks: 2 }));
    const pipe = new LatentPipeline(gpu, dit, { te, adapter: A });
    const P = c.prompts.map((p) => ({ qwenIds: p.qwen, t5Ids: p.t5, t5Weights: p.weights }));
    const keep = [P[0], P[1]];
    const c0 = await pipe.encode(P[0], keep);
    const c1 = await pipe.encode(P[1], keep);
    const c0again = await pipe.encode({ qwenIds: P[0].qwenIds.slice(), t5Ids: P[0].t5Ids.slice(), t5Weights: P[0].t5Weights.slice() }, keep);
    const reused = c0again === c0;
    const stats1 = Object.assign({}, pipe.stats);
    // reference batch: both contexts through prepareContext at once
    const ctxs = [];
    for (const p of P.slice(0, 2)) {
      const hidden = await te.encode(p.qwenIds);
      ctxs.push(await adapt(gpu, A, hidden, p.t5Ids, p.t5Weights));
      hidden.release();
    }
    const both = dit.prepareContext(ctxs);
    const stacked = dit.stackConds([c0, c1]);
    const tc = dit.timeCond(0.6);
    const hw = c.size / 8, per = 16 * hw * hw;
    const lat = [0, 1].map((b) => new TorchGenerator(50 + b).randn(per));
    const vA = await dit.forward(lat, hw, hw, both, tc);
    const vB = await dit.forward(lat, hw, hw, stacked, tc);
    let diffs = 0;
    vA.forEach((va, b) => va.forEach((x, i) => { if (x !== vB[b][i]) diffs++; }));
    stacked.release();
    both.release();
    // a third prompt with the default keep list evicts the other two
    await pipe.encode(P[2]);
    const after = { size: pipe.ctxCache.size, hasP0: pipe.ctxCache.has(JSON.stringify([P[0].qwenIds, P[0].t5Ids, P[0].t5Weights])) };
    tc.release();
    pipe.clearContexts();
    te.release();
    console.log(JSON.stringify({ encode: { reused, stats1, stats: pipe.stats, diffs, n: vA[0].length, after,
      finite: vA.every((v) => v.every((x) => Number.isFinite(x))) } }));
  } else if (c.case === "lnmod") {
    const x = gpu.fromArray(load(c.x), [c.rows, c.cols]);
    const mod = gpu.upload(load(c.mod));
    const y = ops.layernormMod(gpu, x, mod, 0, c.cols, c.cols, !!c.rotate);
    save(c.out, await gpu.read(y));
    if (c.rotate) {
      const q = ops.layernormModQ(gpu, x, mod, 0, c.cols, c.cols);
      save(c.out + ".q", await gpu.read(q.q));
      save(c.out + ".s", await gpu.read(q.s));
    }
  } else if (c.case === "dit") {
    const st = SafeTensors.open(c.weights);
    const dit = AnimaDiT.load(gpu, st, c.blocks);
    const tc = dit.timeCond(c.sigma);
    const ctxs = c.ctx.map((p) => gpu.fromArray(load(p), [c.Lk, 1024]));
    const cond = dit.prepareContext(ctxs);
    const lat = c.latents.map((p) => load(p));
    const h = c.h, w = c.w;
    const blockOut = [];
    const v = await dit.forward(lat, h, w, cond, tc, async (i, x) => {
      if (i === 0) blockOut.push(await gpu.read(x));
    });
    v.forEach((vb, b) => save(c.out + "." + b, vb));
    save(c.out + ".block0", blockOut[0]);
    // which blocks run the stacked q/k/v GEMM (the rest run the three-linear fallback)
    fs.writeFileSync(c.out + ".stacked.json", JSON.stringify(dit.blocks.map((b) => !!b.self.qkv)));
    st.close();
  } else {
    throw new Error("unknown case " + c.case);
  }
  await gpu.sync();
  gpu.destroy();
  console.log(JSON.stringify({ ok: true, case: c.case }));
}

main().catch((e) => {
  process.stderr.write(String(e && e.stack ? e.stack : e) + "\n");
  process.exitCode = 1;
});
