// HIP runtime facade with the call surface of the reference's WebGPU runtime
// (app/gpu/device.js): GPU.create / empty / fromArray / upload / read / flush / sync, the
// size-bucketed buffer pool and a per-op timing profiler. Memory and launches live in the
// ns2 library (lib/libns2.so) behind the N-API addon; this file only keeps JS-side handles.
//
// Ordering: every op is launched on one in-order HIP stream as it is issued, so flush() has
// nothing to submit, and read()/sync() wait for the stream (app/gpu/device.js:206-222).

import { native } from "./native.js";

// A device allocation (the analogue of a GPUBuffer): BigInt address + byte size.
export class DeviceBuffer {
  constructor(ptr, size, pooled = false) {
    this.ptr = ptr;
    this.size = size;
    this.pooled = pooled;
  }
  destroy() {
    if (this.ptr !== null && !this.pooled) native.free(this.ptr);
    this.ptr = null;
  }
}

// app/gpu/device.js:10-24. dtype "f32" (activations) or "f16" (rotated GEMM operands).
export class Tensor {
  constructor(gpu, buf, shape, bytes, dtype = "f32") {
    this.gpu = gpu;
    this.buf = buf;
    this.shape = shape;
    this.bytes = bytes;
    this.dtype = dtype;
  }
  get size() {
    return this.shape.reduce((a, b) => a * b, 1);
  }
  release() {
    if (this.buf) this.gpu.pool.put(this.buf, this.bytes);
    this.buf = null;
  }
}

// Device address of a Tensor / DeviceBuffer, or null.
export function addr(x) {
  if (x === null || x === undefined) return null;
  const b = x.buf !== undefined ? x.buf : x;
  if (!b || b.ptr === null || b.ptr === undefined) throw new Error("use of a released tensor");
  return b.ptr;
}

// app/gpu/device.js:26-57, backed by ns2_pool_* (same bucket rounding).
class BufferPool {
  constructor() {
    this.held = null;
    this.liveBytes = 0;  // bytes of pooled buffers handed out and not yet put back
  }
  static round(bytes) {
    return native.poolRound(bytes);
  }
  get(bytes) {
    const [ptr, size] = native.poolGet(bytes);
    this.liveBytes += size;
    return { buf: new DeviceBuffer(ptr, size, true), size };
  }
  put(buf, size) {
    this.liveBytes -= size;
    if (this.held) this.held.push([buf, size]);
    else native.poolPut(buf.ptr, size);
  }
  // Between holdBegin and holdEnd released buffers are kept out of circulation; holdEnd returns
  // them ([buf, size] pairs) for putAll.
  holdBegin() {
    if (this.held) throw new Error("BufferPool: nested hold");
    this.held = [];
  }
  holdEnd() {
    const h = this.held || [];
    this.held = null;
    return h;
  }
  putAll(list) {
    for (const [buf, size] of list) native.poolPut(buf.ptr, size);
  }
  trim() {
    native.poolTrim();
  }
  get allocated() {
    return native.poolStats().allocated;
  }
  get live() {
    return this.liveBytes;
  }
  get peak() {
    return native.poolStats().peak;
  }
}

export class GPU {
  // app/gpu/device.js:61-81. profile: time every op with stream events.
  static async create({ profile = false, device = 0 } = {}) {
    native.init(device);
    const gpu = new GPU(native.deviceInfo());
    if (profile) gpu.profiler = new Profiler();
    return gpu;
  }

  constructor(info) {
    this.info = info;
    this.profiler = null;
    this.pool = new BufferPool();
    this.maxBinding = Number.MAX_SAFE_INTEGER;
    this.lost = null;
  }

  // ------------------------------------------------------------------ tensors

  empty(shape, dtype = "f32") {
    const bytes = shape.reduce((a, b) => a * b, 1) * (dtype === "f16" ? 2 : 4);
    const { buf, size } = this.pool.get(bytes);
    return new Tensor(this, buf, shape, size, dtype);
  }

  fromArray(arr, shape) {
    const n = shape.reduce((a, b) => a * b, 1);
    if (arr.byteLength > n * 4) {
      throw new Error(`GPU.fromArray: ${arr.byteLength} bytes do not fit shape [${shape}] (${n * 4} bytes)`);
    }
    const t = this.empty(shape);
    this.write(t.buf, arr);
    return t;
  }

  // Copy a typed array into a device buffer at a byte offset; the copy must stay inside the
  // buffer (WebGPU's writeBuffer raises the same validation error).
  write(buf, arr, offset = 0) {
    if (!buf || buf.ptr === null) throw new Error("GPU.write: destination buffer was released");
    if (!(offset >= 0) || offset + arr.byteLength > buf.size) {
      throw new Error(`GPU.write: ${arr.byteLength} bytes at offset ${offset} overrun a ${buf.size}-byte buffer`);
    }
    native.h2d(buf.ptr, arr, offset);
  }

  // Persistent (non-pooled) buffer for weights (app/gpu/device.js:133-139).
  upload(arr) {
    const size = Math.max(16, Math.ceil(arr.byteLength / 16) * 16);
    const ptr = native.malloc(size);
    native.h2d(ptr, arr);
    return new DeviceBuffer(ptr, size, false);
  }

  async read(t, count = t.size) {
    if (!(count >= 0) || count > t.size) {
      throw new Error(`GPU.read: ${count} values requested from a tensor of ${t.size}`);
    }
    const out = new Float32Array(count);
    native.d2h(addr(t), out);
    return out;
  }

  flush() {}

  // Records the launches that fn issues as one HIP graph instead of running them (the
  // replayable analogue of the reference's command-buffer batching, app/gpu/device.js:196-215).
  // fn runs twice: eagerly first, with every release held back, so that the pool afterwards has
  // a free buffer for each tensor fn allocates (and the workspaces their sizes); then under
  // capture, where it allocates nothing new. fn may not read, write or sync. The tensors fn
  // releases during the capture are the graph's own scratch: they stay out of the pool until
  // destroy(), so no live tensor can alias them when the graph is replayed. Returns { result:
  // fn's recorded return value, launch(), destroy() }; a replay reuses the addresses fn saw,
  // so the caller keeps fn's inputs and result alive and refills the inputs in place.
  capture(fn) {
    if (this.profiler) throw new Error("GPU.capture: turn the per-op profiler off first");
    this.pool.holdBegin();
    try {
      const r = fn();
      if (r && typeof r.release === "function") r.release();
    } finally {
      this.pool.putAll(this.pool.holdEnd());
    }
    native.graphBegin();
    this.pool.holdBegin();
    let result;
    try {
      result = fn();
    } catch (e) {
      try { native.graphDestroy(native.graphEnd()); } catch (_) { /* the capture is void anyway */ }
      this.pool.putAll(this.pool.holdEnd());
      throw e;
    }
    let handle;
    try {
      handle = native.graphEnd();
    } catch (e) {
      this.pool.putAll(this.pool.holdEnd());
      throw e;
    }
    const scratch = this.pool.holdEnd();
    return {
      result,
      launch: () => {
        if (handle === null) throw new Error("GPU.capture: launch of a destroyed graph");
        native.graphLaunch(handle);
      },
      destroy: () => {
        if (handle === null) return;
        native.graphDestroy(handle);
        handle = null;
        this.pool.putAll(scratch);
      },
    };
  }

  async sync() {
    native.sync();
  }

  dispatch() {
    throw new Error("GPU.dispatch takes WGSL source; this build launches typed HIP kernels through ops.js");
  }

  // Issue one op; with the profiler on, bracket it with timing events.
  run(name, flops, launch) {
    if (!this.profiler || this.profiler.paused) return launch();
    const [a, b] = this.profiler.next({ name, flops });
    native.eventRecord(a);
    const r = launch();
    native.eventRecord(b);
    return r;
  }
}

// Per-op GPU timings aggregated by name (app/gpu/device.js:234-288).
class Profiler {
  constructor() {
    this.paused = false;  // ops issued while paused are not timed
    this.pending = [];
    this.spare = [];
    this.stats = new Map();
  }
  next(meta) {
    const a = this.spare.pop() || native.eventCreate();
    const b = this.spare.pop() || native.eventCreate();
    this.pending.push({ meta, a, b });
    return [a, b];
  }
  collect() {
    for (const p of this.pending) {
      const ms = native.eventElapsed(p.a, p.b);
      const s = this.stats.get(p.meta.name) || { name: p.meta.name, count: 0, ms: 0, flops: 0 };
      s.count++;
      s.ms += ms;
      s.flops += p.meta.flops || 0;
      this.stats.set(p.meta.name, s);
      this.spare.push(p.a, p.b);
    }
    this.pending = [];
  }
  reset() {
    this.collect();
    this.stats.clear();
  }
  async report() {
    this.collect();
    return [...this.stats.values()].sort((x, y) => y.ms - x.ms);
  }
}

// Split a linear workgroup count into a 2-D grid (app/gpu/device.js:290-295); kept for
// callers of the reference API, HIP grids need no split.
export function grid(n) {
  if (n <= 65535) return [n, 1];
  const y = Math.ceil(n / 65535);
  return [Math.ceil(n / y), y];
}
