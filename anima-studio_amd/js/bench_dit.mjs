// One full DiT step at 1024x1024 through the JS -> N-API -> HIP path: B=2 (CFG cond + uncond),
// 28 blocks, hidden 2048, 16x128 heads, MLP 8192, self + cross attention to 512x1024 contexts,
// seeded random-init weights in the W4A8 "mixed" layout (blocks 0 and 27 int8).
// A step is timeCond(sigma) + forward() (the per-prompt context K/V are cached beforehand, as in
// app/pipeline.js:195-211).  Prints one JSON line.
//
//   node bench_dit.mjs [--size 1024] [--blocks 28] [--mode w4a8|int8|bf16] [--steps 3] [--warmup 1] [--profile]
//                     [--lora-rank R]   (seeded rank-R LoRAs on every block linear, strength 1)
//                     [--generate N [--sampler euler_a] [--cfg 4]]  (also time an N-step sampling run:
//                      the device loop of pipeline.mjs and the reference's host loop)
//                     [--text-encoder N]  (also time Qwen3.encode of N tokens on a 28-layer synthetic
//                      text encoder: causal GQA attention, bf16 linears)
//                     [--vae]  (also time the VAE decode of this size's latent, bf16 and fp32 precision)
//                     [--w4 packed|in-gemm|int8]  (W4 weights kept packed: the large products unpack
//                      them per call into a pooled int8 scratch grid (packed) or inside the GEMM main
//                      loop (in-gemm); int8: converted to their int8 grid once at load.  Bit-identical
//                      products.)
//                     [--in-gemm-too]  (with packed W4: also time the step with the in-GEMM unpack,
//                      reported as w4_in_gemm)
//                     [--no-fuse-qkv]  (the self-attention K / V converted by the attention's own prep
//                      kernel instead of in the QKV GEMM epilogue)
//                     [--unpacked-too]  (with packed W4: also time the step after converting the W4
//                      linears to their int8 grid in place, reported as w4_unpacked)
//                     [--settle-ms 1500]  (after the warmup steps, steps until this much device time
//                      has passed, before anything is timed)
//                     [--graph [--rounds 3]]  (also the forward replayed from a HIP graph recorded
//                      once, ForwardGraph: graph and eager blocks of --steps steps alternate,
//                      medians; dit_step_ms stays the eager step, graph_step_ms the replay)

import { GPU, native } from "./gpu.mjs";
import { SyntheticWeights } from "./weights.mjs";
import { AnimaDiT, ForwardGraph } from "./dit.mjs";
import { linearRegistry, attachLoras, rotatedA } from "./lora.mjs";
import { LatentPipeline } from "./pipeline.mjs";
import { Qwen3 } from "./qwen3.mjs";
import { VAEDecoder, VAE_UPSAMPLES, VAE_DIM } from "./vae.mjs";

function arg(name, def) {
  const i = process.argv.indexOf("--" + name);
  if (i < 0) return def;
  const v = process.argv[i + 1];
  return v === undefined || v.startsWith("--") ? true : v;
}

// Box-Muller over a 32-bit LCG: seeded synthetic latents (host side, like the noise of rng.js).
function normals(n, seed) {
  const out = new Float32Array(n);
  let s = seed >>> 0;
  const u = () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return (s + 1) / 4294967297;
  };
  for (let i = 0; i < n; i += 2) {
    const r = Math.sqrt(-2 * Math.log(u()));
    const t = 2 * Math.PI * u();
    out[i] = r * Math.cos(t);
    if (i + 1 < n) out[i + 1] = r * Math.sin(t);
  }
  return out;
}

async function main() {
  const size = Number(arg("size", 1024));
  const nBlocks = Number(arg("blocks", 28));
  const mode = arg("mode", "w4a8");
  const steps = Number(arg("steps", 3));
  const warmup = Number(arg("warmup", 1));
  const profile = !!arg("profile", false);
  const B = 2, Lk = 512;
  const h = size / 8, w = size / 8;

  const gpu = await GPU.create({ profile });
  const src = new SyntheticWeights(gpu, 1234, { mode, blocks: nBlocks });
  const dit = AnimaDiT.synthetic(gpu, src);
  // --w4 int8: W4 weights converted to their int8 grid at load (bit-identical products, no
  // nibble unpack per GEMM; one byte per weight)
  const w4mode = arg("w4", "packed");
  const unpacked = w4mode === "int8" ? dit.unpackW4() : 0;
  if (w4mode === "in-gemm") native.setW4Path(gpu.ctx, 1);
  if (arg("no-fuse-qkv", false)) dit.fuseQkv = false;
  const ctxs = [0, 1].map((b) => {
    const t = gpu.empty([Lk, 1024]);
    native.fillRandom(gpu.ctx, t.buf, t.size, 4, 77 + b, 1.0, 0.0); // ~N(0,1)
    return t;
  });
  const cond = dit.prepareContext(ctxs);
  const loraRank = Number(arg("lora-rank", 0));
  const loraBufs = [];
  const regs = { dit: linearRegistry(dit), te: null };
  if (loraRank > 0) {
    // one synthetic LoRA module per block linear (stacked q/k/v per part), in the layout loadLora
    // produces: A [r, K], A H for ConvRot targets, B [n, r], scale alpha / r = 1
    const modules = [];
    let seed = 900;
    for (const [name, t] of regs.dit) {
      if (!name.startsWith("blocks_")) continue;
      const A = gpu.empty([loraRank * t.W.K]), B = gpu.empty([t.n * loraRank]);
      native.fillRandom(gpu.ctx, A.buf, A.size, 4, seed++, 0.02, 0.0);
      native.fillRandom(gpu.ctx, B.buf, B.size, 4, seed++, 0.02, 0.0);
      const Ar = t.W.kind === "i8" || t.W.kind === "w4" ? rotatedA(gpu, A, A.size) : null;
      loraBufs.push(A, B);
      if (Ar) loraBufs.push(Ar);
      modules.push({ target: t, A, Ar, B, r: loraRank, alphaScale: 1 });
    }
    attachLoras(regs, [{ lora: { modules }, strength: 1 }]);
  }
  const latents = [normals(16 * h * w, 1), normals(16 * h * w, 2)];
  await gpu.sync();
  process.stderr.write(`bench_dit: model ready (${nBlocks} blocks, ${mode}, W4 ${w4mode}${unpacked ? `: ${unpacked} linears` : ""}), ${(gpu.pool.allocated / 2 ** 30).toFixed(2)} GiB\n`);

  const useGraph = !!arg("graph", false);
  const rounds = Number(arg("rounds", 3));
  let fg = null, latT = null;
  const per = 16 * h * w, host = new Float32Array(B * per);
  if (useGraph) {
    latT = gpu.empty([B, 16, h, w]);
    const tc0 = dit.timeCond(0.9);
    fg = await ForwardGraph.capture(dit, latT, h, w, cond, tc0);
    tc0.release();
  }
  // a step: timeCond, latents up, the forward, velocities back (dit.forward's host work)
  const step = async (eager) => {
    const tc = dit.timeCond(0.9);
    let v;
    if (fg && !eager) {
      latents.forEach((lat, b) => host.set(lat, b * per));
      gpu.write(latT, host);
      const o = await gpu.read(fg.run(tc));
      v = latents.map((_, b) => o.slice(b * per, (b + 1) * per));
    } else {
      v = await dit.forward(latents, h, w, cond, tc);
    }
    tc.release();
    return v;
  };
  let v = null;
  for (let i = 0; i < warmup; i++) v = await step();
  await gpu.sync();
  // settle: keep stepping until the device has run ~settleMs of steps, so that the timed steps
  // see the sustained clocks rather than the ramp after load
  const settleMs = Number(arg("settle-ms", 1500));
  for (let t = 0; t < settleMs; ) {
    gpu.timerStart();
    v = await step();
    t += gpu.timerStop();
  }
  if (gpu.profiler) gpu.profiler.reset();
  // each step timed on its own (HIP events on the library stream around the whole step)
  const timed = async (eager) => {
    const xs = [];
    for (let i = 0; i < steps; i++) {
      gpu.timerStart();
      v = await step(eager);
      xs.push(gpu.timerStop());
    }
    return xs;
  };
  const median = (xs) => xs.slice().sort((a, b) => a - b)[xs.length >> 1];
  let ms, graphMs = null, stepMs;
  if (fg) {
    // graph replays and eager forwards (launched kernel by kernel) in alternating blocks of
    // `steps` steps; medians over every step of the rounds
    await step(true);
    let g = [], e = [];
    for (let r = 0; r < rounds; r++) {
      g = g.concat(await timed(false));
      e = e.concat(await timed(true));
    }
    graphMs = median(g);
    ms = median(e);
    stepMs = e;
  } else {
    stepMs = await timed(false);
    ms = median(stepMs);
  }
  await gpu.sync();
  let finite = true;
  for (const x of v) for (let i = 0; i < x.length; i += 97) if (!Number.isFinite(x[i])) { finite = false; break; }
  const L = (h / 2) * (w / 2);
  // algorithmic FLOPs per step (2*M*N*K GEMMs, 4*Lq*Lk*D*H attention; app/gpu/ops.js:31, 174)
  const M = B * L;
  const perBlock = 2 * M * D_(3 * 2048, 2048) + 2 * M * D_(2048, 2048) * 3 + 2 * M * D_(8192, 2048) * 2 +
    4 * B * L * L * 128 * 16 + 4 * B * L * Lk * 128 * 16;
  const flops = nBlocks * perBlock + 2 * M * 2048 * 68 + 2 * M * 64 * 2048;
  const out = { dit_step_ms: Number(ms.toFixed(3)), step_ms: stepMs.map((x) => Number(x.toFixed(3))), size, blocks: nBlocks, w4: w4mode,
    mode, B, tokens: L, steps, warmup, lora_rank: loraRank, graph: useGraph,
    graph_step_ms: graphMs === null ? null : Number(graphMs.toFixed(3)),
    flops_per_step: flops, tflops: Number((flops / (ms / 1e3) / 1e12).toFixed(2)), finite,
    peak_gib: Number((gpu.pool.peak / 2 ** 30).toFixed(2)) };
  if (gpu.profiler) out.kernels = await gpu.profiler.report();
  const genSteps = Number(arg("generate", 0));
  const note = (what) => process.stderr.write(`bench_dit: ${what}\n`);
  note(`steps done (${ms.toFixed(2)} ms)`);
  if (genSteps > 0) {
    note(`sampling loop, ${genSteps} steps`);
    // a whole sampling run (text encoding and VAE excluded): N DiT steps + the sampler between them
    const pipe = new LatentPipeline(gpu, dit);
    const opts = { cond, width: size, height: size, steps: genSteps, sampler: arg("sampler", "euler_a"),
      cfg: Number(arg("cfg", 4)), seed: 1, scheduler: "simple" };
    await pipe.generate(Object.assign({}, opts, { steps: 1 })); // first-use allocations
    const dev = await pipe.generate(opts);
    // the same run with steps 1.. replayed from a HIP graph of the forward (opts.graph)
    const devg = await pipe.generate(Object.assign({}, opts, { graph: true }));
    const host = await pipe.generateHost(opts);
    pipe.clearTimeCache();
    out.generate = { sampler: opts.sampler, steps: genSteps, cfg: opts.cfg,
      device_ms_per_step: Number(dev.timings.perStep.toFixed(2)),
      device_graph_ms_per_step: Number(devg.timings.perStep.toFixed(2)),
      host_loop_ms_per_step: Number(host.timings.perStep.toFixed(2)) };
  }
  const teTokens = Number(arg("text-encoder", 0));
  if (teTokens > 0) {
    note(`text encoder, ${teTokens} tokens`);
    const te = Qwen3.synthetic(gpu, new SyntheticWeights(gpu, 99), { vocab: 4096 });
    const ids = [];
    for (let i = 0; i < teTokens; i++) ids.push((i * 2654435761) % 4096);
    // three warmup encodes (the first ones of a process run slower: fresh pool buffers, clock ramp)
    for (let i = 0; i < 3; i++) (await te.encode(ids)).release();
    await gpu.sync();
    gpu.timerStart();
    for (let i = 0; i < 5; i++) (await te.encode(ids)).release();
    const teMs = gpu.timerStop() / 5;
    out.text_encoder = { tokens: teTokens, layers: te.layers.length, ms: Number(teMs.toFixed(3)),
      note: "Qwen3.encode: embedding gather on the host, 28 layers, causal GQA 16/8 heads, bf16 linears" };
    te.release();
  }
  if (arg("vae", false)) {
    note("VAE decode");
    // the VAE decoder (Wan 2.1, seeded synthetic weights) on this size's latent, both precisions:
    // the decode of a [16, h, w] latent to a (8h x 8w) image, host conversions included
    const vae = VAEDecoder.synthetic(gpu, new SyntheticWeights(gpu, 77));
    const lat = normals(16 * h * w, 7);
    out.vae = { latent: [16, h, w], image: [8 * h, 8 * w], gflop: Number((vaeFlops(h, w) / 1e9).toFixed(1)) };
    // both precisions warmed up first: the first decodes of a process run their middle stage
    // (the 16384-token attention over a fresh 1 GiB score buffer) several times slower
    for (let i = 0; i < 3; i++) {
      for (const prec of ["bf16", "fp32"]) {
        vae.precision = prec;
        await vae.decode(lat, h, w);
      }
    }
    for (const prec of ["bf16", "fp32"]) {
      vae.precision = prec;
      const ts = [];
      for (let i = 0; i < 3; i++) {
        gpu.timerStart();
        await vae.decode(lat, h, w);
        ts.push(gpu.timerStop());
      }
      const ms = ts.sort((a, b) => a - b)[1];
      out.vae[prec] = { ms: Number(ms.toFixed(2)), "TFLOP/s": Number((vaeFlops(h, w) / ms / 1e9).toFixed(1)) };
    }
  }
  if (arg("in-gemm-too", false) && w4mode === "packed" && mode === "w4a8") {
    note("step with the W4 unpack inside the GEMMs");
    // the same packed weights with the nibbles unpacked inside every GEMM's main loop (eager
    // steps; bit-identical velocities)
    native.setW4Path(gpu.ctx, 1);
    for (let i = 0; i < warmup; i++) await step(true);
    await gpu.sync();
    const xs = await timed(true);
    out.w4_in_gemm = { step_ms: Number(median(xs).toFixed(3)) };
    native.setW4Path(gpu.ctx, 0);
  }
  if (arg("unpacked-too", false) && w4mode === "packed" && mode === "w4a8") {
    note("step with the W4 weights converted to int8");
    // the same step once the W4 linears are converted to their int8 grid in place (after the
    // graph, which holds the packed buffers, is released): bit-identical velocities
    if (fg) {
      fg.release();
      fg = null;
    }
    const n = dit.unpackW4();
    for (let i = 0; i < warmup; i++) await step(true);
    await gpu.sync();
    const xs = await timed(true);
    out.w4_unpacked = { linears: n, step_ms: Number(median(xs).toFixed(3)) };
  }
  console.log(JSON.stringify(out));
  note("done");
  if (fg) fg.release();
  if (latT) latT.release();
  cond.release();
  attachLoras(regs, []);
  for (const t of loraBufs) t.release();
  gpu.destroy();
}

function D_(n, k) {
  return n * k;
}

// algorithmic FLOPs of one VAE decode of an h x w latent (2*M*N*K per convolution / linear, 4*L*L*D
// for the attention)
function vaeFlops(h, w) {
  const conv = (HW, cin, cout) => 2 * HW * cout * 9 * cin;
  const res = (HW, cin, cout) => conv(HW, cin, cout) + conv(HW, cout, cout) + (cin !== cout ? 2 * HW * cout * cin : 0);
  let HW = h * w;
  let f = 2 * HW * 16 * 16 + conv(HW, 16, VAE_DIM) + 2 * res(HW, VAE_DIM, VAE_DIM);
  f += 2 * HW * 3 * VAE_DIM * VAE_DIM + 4 * HW * HW * VAE_DIM + 2 * HW * VAE_DIM * VAE_DIM;
  for (const s of VAE_UPSAMPLES) {
    if (s.up) {
      HW *= 4;
      f += conv(HW, s.up, s.up / 2);
    } else {
      f += res(HW, s[0], s[1]);
    }
  }
  return f + conv(HW, 96, 3);
}

main().catch((e) => {
  process.stderr.write(String(e && e.stack ? e.stack : e) + "\n");
  process.exitCode = 1;
});
