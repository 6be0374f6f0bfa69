// The sampling half of AnimaPipeline.generate (app/pipeline.js:225-293) on the device: initial
// noise, the sigma schedule, per step timeCond -> DiT velocities (cond and uncond batched as B=2)
// -> CFG combine + denoised + sampler update in one kernel (anima_sampler_step), then the latent
// comes back once at the end and, when the pipeline holds a VAE decoder (vae.mjs), is decoded to
// the image as the reference's generate does (pipeline.js:284-292).  The caller passes the
// conditioning made by AnimaDiT.prepareContext ([positive] or, with CFG, [positive, negative]), or
// the per-prompt conditionings of encode() (cached per prompt, as pipeline.js:192-211 caches them).
//
// Noise is drawn on the host with the reference's torch.randn port (rng.mjs), in the reference's
// order, and uploaded; drawing it after the step's DiT work is enqueued overlaps it with that work.
// timeCond results are cached per sigma (they depend only on sigma and on the weights / LoRAs).
// With opts.graph, step 0's forward runs eagerly and, while the device executes it, the forward
// is recorded into a HIP graph (dit.mjs ForwardGraph) that every later step replays with its
// own timeCond.

import { native } from "./gpu.mjs";
import { TorchGenerator } from "./rng.mjs";
import { ForwardGraph, adapt } from "./dit.mjs";
import { SCHEDULERS, SamplerPlan, sample } from "./samplers.mjs";
import { loraGeneration } from "./lora.mjs";

const TIME_CACHE_MAX = 64;

export class LatentPipeline {
  // opts.vae: a VAEDecoder; generate then also returns the decoded image.  opts.te (a Qwen3 text
  // encoder, qwen3.mjs) and opts.adapter (the LLM adapter, dit.mjs) enable encode().
  constructor(gpu, dit, opts) {
    const o = opts || {};
    this.gpu = gpu;
    this.dit = dit;
    this.vae = o.vae || null;
    this.te = o.te || null;
    this.adapter = o.adapter || null;
    this.timeCache = new Map(); // key -> timeCond result (device tensors), in insertion (LRU) order
    this.ctxCache = new Map(); // prompt key -> prepared conditioning (B = 1)
    this.ctxGeneration = loraGeneration();
    this.stats = { timeCondHits: 0, timeCondMisses: 0, encodeHits: 0, encodeMisses: 0 };
  }

  // Prompt -> conditioning ready for the DiT (AnimaPipeline.encode, app/pipeline.js:192-211): token
  // ids -> te.encode -> the LLM adapter -> prepareContext (per-block cross-attention K/V, converted
  // once to the attention's operand layout).  The tokenizer is not part of this build: `prompt` is
  // what the reference's tokenizer.encode returns, { qwenIds, t5Ids, t5Weights }, plus an optional
  // `key` (the prompt text; default: the ids).  Only the prompts in `keep` (keys or prompts; default
  // this one) stay cached -- the reference keeps the positive and negative prompt of the current
  // image, each entry holding every block's K/V -- and attaching LoRAs (a new LoRA generation)
  // clears the cache, as applyLoras -> clearContexts does.  The result belongs to the cache.
  async encode(prompt, keep) {
    if (!this.te || !this.adapter) throw new Error("encode: the pipeline was built without opts.te / opts.adapter");
    const key = promptKey(prompt);
    const keys = (keep || [prompt]).map((k) => (typeof k === "string" ? k : promptKey(k)));
    if (this.ctxGeneration !== loraGeneration()) {
      this.clearContexts();
      this.ctxGeneration = loraGeneration();
    }
    for (const [k, t] of this.ctxCache)
      if (!keys.includes(k)) {
        t.release();
        this.ctxCache.delete(k);
      }
    if (this.ctxCache.has(key)) {
      this.stats.encodeHits++;
      return this.ctxCache.get(key);
    }
    this.stats.encodeMisses++;
    const hidden = await this.te.encode(prompt.qwenIds);
    const ctx = await adapt(this.gpu, this.adapter, hidden, prompt.t5Ids, prompt.t5Weights);
    hidden.release();
    const cond = this.dit.prepareContext([ctx]);
    this.ctxCache.set(key, cond);
    return cond;
  }

  clearContexts() {
    for (const t of this.ctxCache.values()) t.release();
    this.ctxCache.clear();
  }

  // dit.timeCond(sigma), cached.  The key includes the LoRA generation, so attaching LoRAs
  // (which may touch the time embedder and the adaLN modulation) starts a fresh set.
  timeCond(sigma) {
    const key = `${sigma}|${loraGeneration()}`;
    let tc = this.timeCache.get(key);
    if (tc) {
      this.stats.timeCondHits++;
      this.timeCache.delete(key);
      this.timeCache.set(key, tc);
      return tc;
    }
    this.stats.timeCondMisses++;
    tc = this.dit.timeCond(sigma);
    this.timeCache.set(key, tc);
    while (this.timeCache.size > TIME_CACHE_MAX) {
      const [k, old] = this.timeCache.entries().next().value;
      old.release();
      this.timeCache.delete(k);
    }
    return tc;
  }

  clearTimeCache() {
    for (const tc of this.timeCache.values()) tc.release();
    this.timeCache.clear();
  }

  // opts: { cond, cfg = 1, width, height, steps, sampler, seed = 0, shift = 3, scheduler = "simple",
  //         (cond: one batched conditioning, or an array of them such as [encode(pos), encode(neg)])
  //         onStep(i, readDenoised), onProgress({ phase, step, steps, frac }), signal, graph = false,
  //         decode = true (with a VAE) }.
  //         cond.B must be 2 when cfg != 1 (positive, negative), else 1.
  // Progress and cancellation follow app/pipeline.js:226-256: onProgress after every DiT block
  // (after every step when the forward is a graph replay), the device queue drained every 7 blocks
  // so that both stay responsive, and `signal.aborted` checked at the same points, throwing an
  // Error named "AbortError"; the pool is trimmed on the way out, cancelled or not.
  // Returns { latent: Float32Array [16, h, w], image ({ data: RGBA bytes, width, height } or null),
  // sigmas, timings }.
  async generate(opts) {
    // an array of conditionings (e.g. [encode(positive), encode(negative)]) runs as one batch
    if (Array.isArray(opts.cond)) {
      const cond = this.dit.stackConds(opts.cond);
      try {
        return await this.generate(Object.assign({}, opts, { cond }));
      } finally {
        cond.release();
      }
    }
    const gpu = this.gpu;
    const { cond, width, height, steps, sampler, signal } = opts;
    const onProgress = opts.onProgress || (() => {});
    const check = () => {
      if (signal && signal.aborted) {
        const e = new Error("Generation cancelled");
        e.name = "AbortError";
        throw e;
      }
    };
    const cfg = opts.cfg === undefined ? 1 : opts.cfg;
    const seed = opts.seed || 0, shift = opts.shift === undefined ? 3 : opts.shift;
    const guided = cfg !== 1;
    const B = guided ? 2 : 1;
    if (cond.B !== B) throw new Error(`generate: cfg ${cfg} needs ${B} prompt(s) in cond, got ${cond.B}`);
    const h = height / 8, w = width / 8, n = 16 * h * w;
    const t0 = Date.now();
    const sigmas = (SCHEDULERS[opts.scheduler] || SCHEDULERS.simple)(steps, shift);
    const plan = new SamplerPlan(sampler, sigmas, shift);
    const noise0 = new TorchGenerator(seed).randn(n);
    const x = gpu.fromArray(noise0.map((v) => v * sigmas[0]), [1, 16, h, w]);
    const gen = new TorchGenerator(seed); // the sampler's own generator (samplers.js:105)
    const lat = gpu.empty([B, 16, h, w]);
    const old = gpu.empty([n]), oldD = plan.name === "er_sde" ? gpu.empty([n]) : null;
    const den = opts.onStep ? gpu.empty([n]) : null;
    const useGraph = opts.graph === true && plan.steps > 1;
    const nBlocks = this.dit.blocks.length;
    let fg = null;
    // The reference drains the queue every 7 blocks (pipeline.js:255) to keep progress and
    // cancellation responsive.  Here each such point waits for the previous point's mark instead,
    // so the device keeps the last 7 blocks queued while the host enqueues the next ones (a full
    // drain would idle it for the host's share of every chunk).
    let lastMark = null;
    const pace = async () => {
      const m = gpu.mark();
      if (lastMark !== null) await gpu.waitMark(lastMark);
      lastMark = m;
    };
    try {
      check();
      for (let i = 0; i < plan.steps; i++) {
        const st = plan.step(i);
        const tc = this.timeCond(st.sigma);
        for (let b = 0; b < B; b++) gpu.copy(lat.at(b * n), x, n * 4);
        // the step's noise (samplers.js:105-106: one draw per noisy step, in step order) is drawn on the
        // host once the whole forward is enqueued, before the wait, so that it overlaps the
        // device's work on the queued blocks
        let noise = null;
        const onBlock = async (blk) => {
          check();
          onProgress({ phase: "sample", step: i, steps: plan.steps, frac: (i + (blk + 1) / nBlocks) / plan.steps });
          if (blk === nBlocks - 1 && st.noise) noise = gen.randn(n);
          if (blk % 7 === 6) await pace();
        };
        const v = fg ? fg.run(tc) : await this.dit.forwardDevice(lat, h, w, cond, tc, onBlock);
        if (fg) {
          if (st.noise) noise = gen.randn(n);
          await pace();
          check();
          onProgress({ phase: "sample", step: i, steps: plan.steps, frac: (i + 1) / plan.steps });
        }
        const eps = st.noise ? gpu.fromArray(noise || gen.randn(n), [n]) : null;
        native.samplerStep(gpu.ctx, {
          kind: st.kind, n, x: x.buf, v: v.buf, vUncond: guided ? v.at(n) : 0, cfg, sigma: st.sigma,
          final: st.final, stage: st.stage, den: den ? den.buf : 0, old: plan.kind >= 2 ? old.buf : 0,
          oldD: oldD ? oldD.buf : 0, eps: eps ? eps.buf : 0, c: st.c,
        });
        if (!fg) v.release();
        if (eps) eps.release();
        if (opts.onStep) await opts.onStep(i, () => gpu.read(den));
        if (useGraph && !fg) fg = await ForwardGraph.capture(this.dit, lat, h, w, cond, tc, false);
      }
      const latent = await gpu.read(x);
      const ms = Date.now() - t0;
      let image = null;
      let decodeMs = 0;
      if (this.vae && opts.decode !== false) {
        check();
        const tv = Date.now();
        onProgress({ phase: "decode", frac: 0 });
        image = await this.vae.decode(latent, h, w, (f) => onProgress({ phase: "decode", frac: f }));
        decodeMs = Date.now() - tv;
      }
      return { latent, image, sigmas, timings: { sample: ms, perStep: ms / plan.steps, decode: decodeMs,
        total: ms + decodeMs } };
    } finally {
      if (fg) fg.release();
      for (const t of [x, lat, old, oldD, den]) if (t) t.release();
      // free pooled activations so that idle device memory is the weights (also after a cancel)
      try {
        await gpu.sync();
      } catch (e) {
        // a device error is reported by the call that hit it
      }
      gpu.pool.trim();
    }
  }

  // The same sampling with the reference's host loop: velocities come back every step, and CFG,
  // the denoised estimate and the sampler update run over Float32Arrays (pipeline.js:276-283,
  // samplers.js:104-218).  For parity checks and as the drop-in's baseline.
  async generateHost(opts) {
    const { cond, width, height, steps, sampler } = opts;
    const cfg = opts.cfg === undefined ? 1 : opts.cfg;
    const seed = opts.seed || 0, shift = opts.shift === undefined ? 3 : opts.shift;
    const guided = cfg !== 1;
    if (cond.B !== (guided ? 2 : 1)) throw new Error(`generateHost: cfg ${cfg} needs ${guided ? 2 : 1} prompt(s)`);
    const h = height / 8, w = width / 8, n = 16 * h * w;
    const t0 = Date.now();
    const sigmas = (SCHEDULERS[opts.scheduler] || SCHEDULERS.simple)(steps, shift);
    const noise0 = new TorchGenerator(seed).randn(n);
    const x0 = noise0.map((v) => v * sigmas[0]);
    const denoise = async (xin, sigma) => {
      const tc = this.timeCond(sigma);
      const vs = await this.dit.forward(guided ? [xin, xin] : [xin], h, w, cond, tc);
      const v = vs[0];
      if (guided) {
        const vn = vs[1];
        for (let j = 0; j < n; j++) v[j] = vn[j] + cfg * (v[j] - vn[j]);
      }
      const den = new Float32Array(n);
      for (let j = 0; j < n; j++) den[j] = xin[j] - sigma * v[j];
      return den;
    };
    const latent = await sample(sampler, denoise, x0, sigmas, { seed, shift });
    const ms = Date.now() - t0;
    return { latent, sigmas, timings: { sample: ms, perStep: ms / (sigmas.length - 1) } };
  }
}

function promptKey(p) {
  if (p.key !== undefined) return String(p.key);
  return JSON.stringify([p.qwenIds, p.t5Ids, p.t5Weights]);
}
