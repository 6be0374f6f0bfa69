// LoRA side paths for the DiT linears (app/lora.js:1-149): each targeted linear W gets entries
// { A: [r, K] f32, B: [n, r] f32, r, scale, off, n } and ops.linear adds
// scale * B (A x) to its output before the activation / gate (ops.js:55-62, 70-87).
//
// Files: PEFT names ("<prefix><module>.lora_A.weight" / ".lora_B.weight") or kohya names
// ("lora_unet_<module with underscores>.lora_down.weight" / ".lora_up.weight" + ".alpha"),
// matched against the model's linears by module name with dots and underscores equivalent.
// LoKr / LoHa / DoRA tensors are counted as unsupported and skipped.  A ConvRot (i8 / w4) layer
// may hold only the rotated input x H, and x A^T = (x H)(A H)^T, so for those layers A H is also
// made once at load time (Ar), on the device, with the same per-256-group Hadamard as the
// activations.  This build runs the DiT only, so text-encoder modules never match.

import { SafeTensors } from "./weights.mjs";
import { native } from "./gpu.mjs";
import { stackLora, releaseLoraStack, splitPlanes, fuseLora, releaseLoraFused } from "./ops.mjs";

const needsRotation = (W) => W.kind === "i8" || W.kind === "w4";
const norm = (name) => name.replace(/\./g, "_");

const SUFFIXES = [
  [".lora_A.weight", "A"], [".lora_B.weight", "B"],
  [".lora_down.weight", "A"], [".lora_up.weight", "B"],
  [".alpha", "alpha"],
];
const TE_PREFIXES = ["lora_te_", "lora_te1_", "text_encoder.", "text_encoders.qwen3_06b.transformer.", "te."];
const DIT_PREFIXES = ["lora_unet_", "model.diffusion_model.", "diffusion_model.", "base_model.model.", "transformer.", "unet."];
const UNSUPPORTED = /(lokr_|hada_|\.dora_scale|\.diff$|\.diff_b$|\.w_norm|\.b_norm)/;
const ANIMA_MODULE = /^(blocks_\d+_|llm_adapter_|x_embedder_|t_embedder_|final_layer_|(model_)?layers_\d+_)/;

function suffixOf(key) {
  for (const s of SUFFIXES) if (key.endsWith(s[0])) return s;
  return null;
}

function stripPrefix(module) {
  for (const p of TE_PREFIXES) if (module.startsWith(p)) return { name: module.slice(p.length), te: true };
  for (const p of DIT_PREFIXES) if (module.startsWith(p)) return { name: module.slice(p.length), te: false };
  return { name: module, te: false };
}

// Tensor-name survey of a LoRA file (app/lora.js:33-47): is it a LoRA, how many modules, how
// many carry Anima module names, how many tensors are of unsupported kinds.
export function inspectLoraKeys(keys) {
  const modules = new Set();
  let unsupported = 0;
  for (const key of keys) {
    if (UNSUPPORTED.test(key)) {
      unsupported++;
      continue;
    }
    const suf = suffixOf(key);
    if (suf && suf[1] !== "alpha") modules.add(key.slice(0, -suf[0].length));
  }
  let anima = 0;
  for (const m of modules) if (ANIMA_MODULE.test(norm(stripPrefix(m).name))) anima++;
  return { lora: modules.size > 0, modules: modules.size, anima, unsupported };
}

// normalized module name -> { W, off, n } for every linear reachable from a model object
// (app/lora.js:51-69); stacked weights register each of their parts.
export function linearRegistry(root) {
  const reg = new Map();
  const seen = new Set();
  const walk = (o) => {
    if (!o || typeof o !== "object" || seen.has(o) || ArrayBuffer.isView(o) || o instanceof SafeTensors) return;
    seen.add(o);
    if (o.kind && o.buf && o.N && o.K) {
      if (o.parts) for (const p of o.parts) reg.set(norm(p.name), { W: o, off: p.off, n: p.n });
      else if (o.name) reg.set(norm(o.name), { W: o, off: 0, n: o.N });
      return;
    }
    for (const k of Object.keys(o)) if (k !== "gpu" && k !== "st") walk(o[k]);
  };
  walk(root);
  return reg;
}

function findTarget(module, regs) {
  const { name, te } = stripPrefix(module);
  const key = norm(name);
  for (const reg of te ? [regs.te] : [regs.dit, regs.te]) {
    if (!reg) continue;
    if (reg.has(key)) return reg.get(key);
    if (reg.has("model_" + key)) return reg.get("model_" + key);
  }
  return null;
}

// Loads a LoRA safetensors file for the registries { dit, te } (app/lora.js:104-135).  Returns
// { modules: [{ target, A, B, r, alphaScale }], matched, total, unsupported, skipped }.
export function loadLora(gpu, path, regs) {
  const st = SafeTensors.open(path);
  try {
    const groups = new Map();
    let unsupported = 0;
    for (const key of Object.keys(st.header)) {
      if (UNSUPPORTED.test(key)) {
        unsupported++;
        continue;
      }
      const suf = suffixOf(key);
      if (!suf) continue;
      const module = key.slice(0, -suf[0].length);
      if (!groups.has(module)) groups.set(module, {});
      groups.get(module)[suf[1]] = key;
    }
    const modules = [];
    let skipped = 0;
    for (const [module, keys] of groups) {
      if (!keys.A || !keys.B) {
        skipped++;
        continue;
      }
      const target = findTarget(module, regs);
      const aShape = st.info(keys.A).shape, bShape = st.info(keys.B).shape;
      const r = aShape[0];
      if (!target || aShape[1] !== target.W.K || bShape[0] !== target.n || bShape[1] !== r) {
        skipped++;
        continue;
      }
      const A = gpu.upload(st.f32(keys.A));
      const Ar = needsRotation(target.W) ? rotatedA(gpu, A, r * target.W.K) : null;
      const B = gpu.upload(st.f32(keys.B));
      const alpha = keys.alpha ? st.f32(keys.alpha)[0] : null;
      modules.push({ target, A, Ar, B, r, alphaScale: alpha ? alpha / r : 1 });
    }
    return { modules, matched: modules.length, total: groups.size, unsupported, skipped };
  } finally {
    st.close();
  }
}

// A H: each row of A through the per-256-group Hadamard of the ConvRot activations.
export function rotatedA(gpu, A, n) {
  const Ar = gpu.empty([n]);
  native.hadamard(gpu.ctx, A.buf || A, Ar.buf, n);
  return Ar;
}

export function destroyLora(L) {
  for (const m of L.modules) {
    m.A.release();
    if (m.Ar) m.Ar.release();
    m.B.release();
  }
}

// Replaces every side path in the registries with the given [{ lora, strength }]
// (app/lora.js:140-149).  A linear with several entries (q/k/v parts, stacked LoRAs) gets its A
// matrices stacked on the device so that one product reads the shared input, and every matrix
// gets its three bf16 planes for the split-product kernels; attachLoras(regs, []) releases both.
let generation = 0;
// Counts attachLoras calls: results cached across calls (timeCond) key on it.
export function loraGeneration() {
  return generation;
}

export function attachLoras(regs, active) {
  generation++;
  const ws = new Set();
  for (const reg of [regs.dit, regs.te]) if (reg) for (const { W } of reg.values()) ws.add(W);
  for (const W of ws) {
    releaseLoraStack(W);
    releaseLoraFused(W);
    if (W.lora) for (const e of W.lora) if (e.owned) for (const t of e.owned) t.release();
    W.lora = [];
  }
  for (const { lora, strength } of active) {
    if (!strength) continue;
    for (const m of lora.modules) {
      const gpu = m.A.gpu, K = m.target.W.K;
      // bf16 planes of the matrices for the split-product kernels (freed on the next attach)
      const As = splitPlanes(gpu, m.A, m.r * K), Ars = m.Ar ? splitPlanes(gpu, m.Ar, m.r * K) : null;
      const Bs = m.r % 8 === 0 ? splitPlanes(gpu, m.B, m.target.n * m.r) : null;
      m.target.W.lora.push({ A: m.A, Ar: m.Ar, B: m.B, As, Ars, Bs, owned: [As, Ars, Bs].filter((t) => t), r: m.r,
        scale: strength * m.alphaScale, off: m.target.off, n: m.target.n });
    }
  }
  for (const W of ws) {
    if (!W.lora.length) continue;
    // quantized weights: the A stack and the B factor for the GEMM epilogue (fuseLora); others:
    // the A stack of the separate products
    if (needsRotation(W)) fuseLora(W.lora[0].A.gpu, W);
    else if (W.lora.length > 1) stackLora(W.lora[0].A.gpu, W);
  }
}
