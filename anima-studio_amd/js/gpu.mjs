// GPU runtime facade over the N-API addon: the surface of the reference's app/gpu/device.js
// (GPU.create, empty, fromArray, write, upload, read, flush, sync, pool, profiler, Tensor, grid)
// backed by one HIP stream on an MI355X instead of a WebGPU queue.
// Node-12 syntax only (no ?. / ??, no class fields).

import { createRequire } from "module";

const require = createRequire(import.meta.url);
export const native = require("./anima.node");

const ESIZE = { f32: 4, i32: 4, bf16: 2, u16: 2, i8: 1, u8: 1 };
const ARRAY = { f32: Float32Array, i32: Int32Array, bf16: Uint16Array, u16: Uint16Array, i8: Int8Array, u8: Uint8Array };

function dtypeOf(arr) {
  if (arr instanceof Float32Array) return "f32";
  if (arr instanceof Int32Array) return "i32";
  if (arr instanceof Uint16Array) return "u16";
  if (arr instanceof Int8Array) return "i8";
  if (arr instanceof Uint8Array) return "u8";
  throw new Error("unsupported typed array " + (arr && arr.constructor && arr.constructor.name));
}

// Device tensor (app/gpu/device.js:10-24).  `buf` is the device address (a Number).  An owning
// tensor holds `handle`, the addon's finalizer-backed owner of the buffer: release() returns the
// buffer to the pool at once; a tensor dropped without release() returns it when the garbage
// collector reclaims the handle (as WebGPU reclaims an unreferenced GPUBuffer).
export class Tensor {
  constructor(gpu, ptr, shape, bytes, dtype, handle) {
    this.gpu = gpu;
    this.buf = ptr;
    this.shape = shape;
    this.bytes = bytes;
    this.dtype = dtype || "f32";
    this.handle = handle || null;
  }
  get size() {
    return this.shape.reduce((a, b) => a * b, 1);
  }
  // device address of element i
  at(i) {
    return this.buf + i * ESIZE[this.dtype];
  }
  // non-owning view of elements [i, i + prod(shape)); it keeps the owning tensor reachable (so
  // the buffer outlives the view), and its release() only drops that reference
  view(i, shape) {
    const t = new Tensor(this.gpu, this.at(i), shape, shape.reduce((a, b) => a * b, 1) * ESIZE[this.dtype], this.dtype);
    t.owner = this.owner || this;
    t.release = () => {
      t.buf = 0;
      t.owner = null;
    };
    return t;
  }
  release() {
    if (this.handle) native.release(this.handle);
    this.handle = null;
    this.buf = 0;
  }
  destroy() {
    this.release();
  }
}

// BufferPool view (app/gpu/device.js:26-57): the pool itself lives in the C runtime.
class Pool {
  constructor(gpu) {
    this.gpu = gpu;
  }
  get allocated() {
    return native.memStats(this.gpu.ctx).allocated;
  }
  get peak() {
    return native.memStats(this.gpu.ctx).peak;
  }
  trim() {
    native.trim(this.gpu.ctx);
  }
}

// Per-kernel timings aggregated by name (app/gpu/device.js:234-288).
class Profiler {
  constructor(gpu) {
    this.gpu = gpu;
  }
  async report() {
    return JSON.parse(native.profileReport(this.gpu.ctx));
  }
  reset() {
    native.profileReset(this.gpu.ctx);
  }
}

export class GPU {
  // GPU.create (app/gpu/device.js:61-81); profile: time every kernel with HIP events.
  static async create(opts) {
    const o = opts || {};
    const gpu = new GPU(native.init(o.device || 0));
    if (o.profile) {
      native.profileEnable(gpu.ctx, true);
      gpu.profiler = new Profiler(gpu);
    }
    return gpu;
  }

  constructor(ctx) {
    this.ctx = ctx;
    this.profiler = null;
    // adapter limits in WebGPU's names (app/gpu/device.js:83-88): HIP caps neither one buffer nor
    // one binding below the device memory, so maxBinding is the device's global memory
    this.limits = native.deviceLimits(ctx);
    this.info = { vendor: "AMD", architecture: this.limits.architecture.split(":")[0], description: "MI355X (HIP)" };
    this.maxBinding = Math.min(this.limits.maxStorageBufferBindingSize, this.limits.maxBufferSize);
    this.pool = new Pool(this);
  }

  empty(shape, dtype) {
    const dt = dtype || "f32";
    const bytes = shape.reduce((a, b) => a * b, 1) * ESIZE[dt];
    const h = native.allocHandle(this.ctx, bytes);
    return new Tensor(this, native.handleAddr(h), shape, bytes, dt, h);
  }

  fromArray(arr, shape) {
    const t = this.empty(shape || [arr.length], dtypeOf(arr));
    native.h2d(this.ctx, t.buf, arr);
    return t;
  }

  write(buf, arr, offset) {
    native.h2d(this.ctx, (buf.buf || buf) + (offset || 0), arr);
  }

  // Persistent buffer for weights (app/gpu/device.js:134-139); a Tensor with release().
  upload(arr) {
    return this.fromArray(arr, [arr.length]);
  }

  async read(t, count) {
    const n = count === undefined ? t.size : count;
    const out = new ARRAY[t.dtype](n);
    native.d2h(this.ctx, t.buf, out);
    return out;
  }

  copy(dst, src, bytes) {
    native.d2d(this.ctx, dst.buf || dst, src.buf || src, bytes);
  }

  // Work is submitted to the HIP stream at enqueue time.
  flush() {}

  async sync() {
    native.sync(this.ctx);
  }

  // A point in the queue (its ticket) and the wait for it: `await gpu.waitMark(t)` returns when
  // the work enqueued before mark t has finished, with device errors surfaced as by sync().
  mark() {
    return native.mark(this.ctx);
  }

  async waitMark(t) {
    native.waitMark(this.ctx, t);
  }

  timerStart() {
    native.timerStart(this.ctx);
  }

  timerStop() {
    return native.timerStop(this.ctx);
  }

  destroy() {
    native.destroy(this.ctx);
    this.ctx = null;
  }
}

// Split a linear workgroup count into a 2D grid (app/gpu/device.js:291-295); kept for callers.
export function grid(n) {
  if (n <= 65535) return [n, 1];
  const y = Math.ceil(n / 65535);
  return [Math.ceil(n / y), y];
}
