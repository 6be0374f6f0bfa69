// Weight sources for the DiT: a safetensors reader with the comfy_quant linear mapping of
// app/weights.js (linearWeights, concatLinears), and a seeded synthetic source that creates the
// same objects directly on the device (benchmarks; no checkpoint ships with this build).
//
// Linear weight objects (app/weights.js:1-4):
//   { kind: "bf16" | "i8" | "w4", N, K, buf, scale?, srel?, codebook?, codebookData?, bias?, name }
// with device Tensors in buf / scale / srel / codebook / bias.

import fs from "fs";
import { native } from "./gpu.mjs";

const BYTES = { F32: 4, BF16: 2, F16: 2, I8: 1, U8: 1, F8_E4M3: 1, I32: 4, I64: 8, F64: 8 };

function bf16ToF32(u8) {
  const u16 = new Uint16Array(u8.buffer, u8.byteOffset, u8.byteLength / 2);
  const out = new Float32Array(u16.length);
  const o32 = new Uint32Array(out.buffer);
  for (let i = 0; i < u16.length; i++) o32[i] = u16[i] << 16;
  return out;
}

function f16ToF32(u8) {
  const u16 = new Uint16Array(u8.buffer, u8.byteOffset, u8.byteLength / 2);
  const out = new Float32Array(u16.length);
  for (let i = 0; i < u16.length; i++) {
    const h = u16[i];
    const s = h & 0x8000 ? -1 : 1;
    const e = (h >> 10) & 31;
    const m = h & 1023;
    out[i] = e === 0 ? s * m * Math.pow(2, -24) : e === 31 ? (m ? NaN : s * Infinity) : s * (1 + m / 1024) * Math.pow(2, e - 15);
  }
  return out;
}

// safetensors: 8-byte little-endian header length, JSON header, then the data block.
export class SafeTensors {
  static open(path, prefix) {
    const fd = fs.openSync(path, "r");
    const head = Buffer.alloc(8);
    fs.readSync(fd, head, 0, 8, 0);
    const n = Number(head.readBigUInt64LE(0));
    const hb = Buffer.alloc(n);
    fs.readSync(fd, hb, 0, n, 8);
    const header = JSON.parse(hb.toString("utf8"));
    delete header.__metadata__;
    return new SafeTensors(fd, header, 8 + n, prefix || "");
  }

  constructor(fd, header, dataStart, prefix) {
    this.fd = fd;
    this.header = header;
    this.dataStart = dataStart;
    this.prefix = prefix;
  }

  close() {
    fs.closeSync(this.fd);
  }

  has(name) {
    return (this.prefix + name) in this.header;
  }

  info(name) {
    const t = this.header[this.prefix + name];
    if (!t) throw new Error(`missing tensor ${this.prefix + name}`);
    return t;
  }

  bytes(name) {
    const t = this.info(name);
    const a = t.data_offsets[0], b = t.data_offsets[1];
    const buf = Buffer.alloc(b - a);
    let done = 0;
    while (done < buf.length) {
      const r = fs.readSync(this.fd, buf, done, buf.length - done, this.dataStart + a + done);
      if (r <= 0) throw new Error(`short read of ${name}`);
      done += r;
    }
    return new Uint8Array(buf.buffer, buf.byteOffset, buf.length);
  }

  f32(name) {
    const t = this.info(name);
    const u8 = this.bytes(name);
    if (t.dtype === "F32") return new Float32Array(u8.slice().buffer);
    if (t.dtype === "BF16") return bf16ToF32(u8.slice());
    if (t.dtype === "F16") return f16ToF32(u8.slice());
    throw new Error(`unsupported dtype ${t.dtype} for ${name}`);
  }

  vector(gpu, name) {
    return gpu.upload(this.f32(name));
  }

  // Rows `ids` of a 2D table (the token embedding) as one Float32Array [ids.length][dim],
  // read row by row (app/weights.js:74-103): F32 / BF16 / F16, or a comfy_quant per-row int8
  // table whose value is q * weight_scale[row].
  async rows(name, ids) {
    const base = name.slice(0, -"weight".length);
    const t = this.info(name);
    const dim = t.shape[1];
    const out = new Float32Array(ids.length * dim);
    const quant = this.has(base + "comfy_quant");
    if (quant && t.dtype !== "I8") throw new Error(`unsupported quantized embedding ${base}`);
    const scales = quant ? this.f32(base + "weight_scale") : null;
    const rowBytes = dim * BYTES[t.dtype];
    const buf = Buffer.alloc(rowBytes);
    ids.forEach((id, i) => {
      if (id < 0 || id >= t.shape[0]) throw new Error(`token id ${id} outside ${name} [${t.shape}]`);
      const r = fs.readSync(this.fd, buf, 0, rowBytes, this.dataStart + t.data_offsets[0] + id * rowBytes);
      if (r !== rowBytes) throw new Error(`short read of ${name} row ${id}`);
      const u8 = new Uint8Array(buf.buffer.slice(buf.byteOffset, buf.byteOffset + rowBytes));
      if (quant) {
        const q = new Int8Array(u8.buffer);
        for (let j = 0; j < dim; j++) out[i * dim + j] = q[j] * scales[id];
      } else {
        out.set(t.dtype === "BF16" ? bf16ToF32(u8) : t.dtype === "F16" ? f16ToF32(u8) : new Float32Array(u8.buffer), i * dim);
      }
    });
    return out;
  }

  linear(gpu, base) {
    const W = this.linearWeights(gpu, base);
    W.name = base.replace(/\.$/, "");
    return W;
  }

  // comfy_quant -> { kind: i8 | w4 }, else bf16 (app/weights.js:118-147)
  linearWeights(gpu, base) {
    const w = this.info(base + "weight");
    const bias = this.has(base + "bias") ? this.vector(gpu, base + "bias") : null;
    if (this.has(base + "comfy_quant")) {
      const meta = JSON.parse(Buffer.from(this.bytes(base + "comfy_quant")).toString("utf8"));
      const N = w.shape[0];
      if (!meta.convrot) throw new Error(`${base}: only ConvRot-quantized linears are supported`);
      if (meta.format === "int8_tensorwise") {
        return { kind: "i8", N, K: w.shape[1], buf: gpu.upload(new Int8Array(this.bytes(base + "weight").slice().buffer)),
          scale: this.vector(gpu, base + "weight_scale"), bias };
      }
      if (meta.format === "asym_w4a8_int8") {
        const codebookData = this.f32(base + "weight_codebook");
        return {
          kind: "w4", N, K: w.shape[1] * 2,
          buf: gpu.upload(this.bytes(base + "weight").slice()),
          srel: gpu.upload(this.bytes(base + "weight_s_rel").slice()),
          scale: this.vector(gpu, base + "weight_s_channel"),
          codebook: gpu.upload(codebookData),
          codebookData,
          bias,
        };
      }
      throw new Error(`unsupported quant format ${meta.format}`);
    }
    if (w.dtype !== "BF16") throw new Error(`expected bf16 weight for ${base}, got ${w.dtype}`);
    const N = w.shape[0];
    const K = w.shape.slice(1).reduce((a, b) => a * b, 1);
    return { kind: "bf16", N, K, buf: gpu.upload(new Uint16Array(this.bytes(base + "weight").slice().buffer)), bias };
  }
}

// Stack linears sharing an input into one [sum N, K] weight (app/weights.js:152-189): rows and
// per-row scales concatenate; w4 also needs one shared codebook.  Returns null otherwise.
export function concatLinears(gpu, Ws) {
  const kind = Ws[0].kind, K = Ws[0].K;
  if (!Ws.every((w) => w.kind === kind && w.K === K && !w.bias)) return null;
  if (kind === "w4") {
    const cb = Ws[0].codebookData;
    if (!Ws.every((w) => w.codebookData.every((v, i) => v === cb[i]))) return null;
  }
  const bytes = {
    buf: (n) => (kind === "bf16" ? n * K * 2 : kind === "i8" ? n * K : (n * K) / 2),
    scale: (n) => n * 4,
    srel: (n) => (n * K) / 16,
  };
  const dtype = { buf: kind === "bf16" ? "u16" : kind === "i8" ? "i8" : "u8", scale: "f32", srel: "u8" };
  const fields = kind === "bf16" ? ["buf"] : kind === "i8" ? ["buf", "scale"] : ["buf", "scale", "srel"];
  const N = Ws.reduce((a, w) => a + w.N, 0);
  const out = { kind, K, N, parts: [] };
  let colOff = 0;
  for (const w of Ws) { out.parts.push({ name: w.name, off: colOff, n: w.N }); colOff += w.N; }
  for (const f of fields) {
    const total = bytes[f](N);
    const esz = dtype[f] === "f32" ? 4 : dtype[f] === "u16" ? 2 : 1;
    const dst = gpu.empty([total / esz], dtype[f]);
    let off = 0;
    for (const w of Ws) {
      gpu.copy(dst.buf + off, w[f], bytes[f](w.N));
      off += bytes[f](w.N);
    }
    out[f] = dst;
  }
  if (kind === "w4") {
    out.codebook = Ws[0].codebook;
    out.codebookData = Ws[0].codebookData;
  }
  for (const w of Ws) for (const f of fields) w[f].release();
  for (const w of Ws.slice(1)) if (kind === "w4") w.codebook.release();
  return out;
}

// Lloyd-Max 16-level codebook of tools/quant.py:22-25 (comfy_kitchen _FIXED_LUT).
export const FIXED_LUT = [-0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
  0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671];

const FILL = { u8: 0, i8n: 1, f32: 2, bf16: 3, f32n: 4 };

// 32-bit FNV-1a of a tensor name: per-tensor seed offset of the synthetic source.
function nameHash(s) {
  let h = 0x811c9dc5;
  for (let i = 0; i < s.length; i++) {
    h ^= s.charCodeAt(i);
    h = Math.imul(h, 0x01000193) >>> 0;
  }
  return h;
}

// Seeded random-init weights in the checkpoint formats, generated on the device.
//   int8:  round(N(0, 40^2)) clipped to +-127 (Irwin-Hall), weight_scale U(0.5,1.5)/(127 sqrt(K))
//   w4:    codes U{0..255} bytes, s_rel e4m3 bytes 0x60..0x6f (32..120), s_channel as int8 scale,
//          codebook FIXED_LUT
//   bf16:  U(-a, a), a = gain * sqrt(3 / K)
// Layer formats follow tools/build_assets.py:68, 119: DiT block linears are int8, or W4 for the
// inner blocks in "w4a8" (mixed) mode; everything else bf16.
export class SyntheticWeights {
  constructor(gpu, seed, opts) {
    const o = opts || {};
    this.gpu = gpu;
    this.seed = seed;
    this.mode = o.mode || "w4a8";
    this.nBlocks = o.blocks || 28;
  }

  seedOf(name) {
    return (this.seed * 1000003 + nameHash(name)) % 9007199254740881;
  }

  fill(t, kind, name, lo, hi) {
    native.fillRandom(this.gpu.ctx, t.buf, t.size, FILL[kind], this.seedOf(name), lo, hi);
    return t;
  }

  vector(gpu, name, n, lo, hi) {
    return this.fill(gpu.empty([n]), "f32", name, lo === undefined ? 0.98 : lo, hi === undefined ? 1.02 : hi);
  }

  quantKind(block) {
    if (this.mode === "bf16") return "bf16";
    if (this.mode === "int8") return "i8";
    return block > 0 && block < this.nBlocks - 1 ? "w4" : "i8";
  }

  // A block linear [N, K] in the block's format.
  blockLinear(gpu, name, N, K, block) {
    const kind = this.quantKind(block);
    if (kind === "bf16") return this.bf16Linear(gpu, name, N, K, 1.0);
    const scale = this.fill(gpu.empty([N]), "f32", name + ".scale", 0.5 / (127 * Math.sqrt(K)), 1.5 / (127 * Math.sqrt(K)));
    if (kind === "i8") {
      return { kind, N, K, name, buf: this.fill(gpu.empty([N * K], "i8"), "i8n", name, 40, 0), scale };
    }
    const codebookData = new Float32Array(FIXED_LUT);
    return {
      kind, N, K, name, scale, codebookData,
      buf: this.fill(gpu.empty([(N * K) / 2], "u8"), "u8", name, 0, 255),
      srel: this.fill(gpu.empty([(N * K) / 16], "u8"), "u8", name + ".srel", 0x60, 0x6f),
      codebook: gpu.upload(codebookData),
    };
  }

  bf16Linear(gpu, name, N, K, gain) {
    const a = gain * Math.sqrt(3 / K);
    return { kind: "bf16", N, K, name, buf: this.fill(gpu.empty([N * K], "bf16"), "bf16", name, -a, a) };
  }
}
