// Weight loading for the Node host: a safetensors reader over a local file with the interface
// the model code uses (has / info / vector / linear; app/weights.js:41-133), and the linear
// weight objects of the reference: { kind: "i8" | "bf16", N, K, buf, scale?, bias?, name }.
//
// int8 layers use ComfyUI's comfy_quant layout written by tools/build_assets.py: `weight` I8
// [N, K], `weight_scale` F32 [N, 1] and `comfy_quant` (U8 JSON) with format
// "int8_tensorwise" and convrot = true; any other quantization is rejected
// (app/weights.js:127-131). bf16 weights are uploaded as raw bf16 and decoded in the GEMM.

import fs from "fs";
import { addr } from "./device.js";
import { native, EW } from "./native.js";

const BYTES = { F32: 4, F16: 2, BF16: 2, I8: 1, U8: 1, I32: 4, I64: 8 };

function bf16ToF32(u8) {
  const src = new Uint16Array(u8.buffer, u8.byteOffset, u8.byteLength / 2);
  const out = new Float32Array(src.length);
  const bits = new Uint32Array(out.buffer);
  for (let i = 0; i < src.length; i++) bits[i] = src[i] << 16;
  return out;
}

function f16ToF32(u8) {
  const src = new Uint16Array(u8.buffer, u8.byteOffset, u8.byteLength / 2);
  const out = new Float32Array(src.length);
  for (let i = 0; i < src.length; i++) {
    const h = src[i];
    const s = h & 0x8000 ? -1 : 1;
    const e = (h >> 10) & 0x1f;
    const m = h & 0x3ff;
    out[i] = e === 0 ? s * m * 2 ** -24 : e === 31 ? (m ? NaN : s * Infinity) : s * (1 + m / 1024) * 2 ** (e - 15);
  }
  return out;
}

function f32ToBf16(f) {
  // round to nearest even
  const bits = new Uint32Array(f.buffer, f.byteOffset, f.length);
  const out = new Uint16Array(f.length);
  for (let i = 0; i < f.length; i++) {
    const b = bits[i];
    out[i] = (b + 0x7fff + ((b >>> 16) & 1)) >>> 16;
  }
  return out;
}

export class SafeTensors {
  static async open(path) {
    return new SafeTensors(path);
  }

  constructor(path) {
    this.path = path;
    this.fd = fs.openSync(path, "r");
    const head = Buffer.alloc(8);
    fs.readSync(this.fd, head, 0, 8, 0);
    const n = Number(head.readBigUInt64LE(0));
    const json = Buffer.alloc(n);
    fs.readSync(this.fd, json, 0, n, 8);
    this.header = JSON.parse(json.toString("utf8"));
    this.metadata = this.header.__metadata__ || {};
    delete this.header.__metadata__;
    this.dataStart = 8 + n;
  }

  close() {
    if (this.fd !== null) fs.closeSync(this.fd);
    this.fd = null;
  }

  has(name) {
    return Object.prototype.hasOwnProperty.call(this.header, name);
  }

  info(name) {
    const t = this.header[name];
    if (!t) throw new Error(`missing tensor ${name}`);
    return t;
  }

  // Raw bytes of a tensor (a fresh, 8-byte aligned buffer).
  async bytes(name) {
    const t = this.info(name);
    const [a, b] = t.data_offsets;
    const u8 = new Uint8Array(new ArrayBuffer(b - a));
    let done = 0;
    while (done < u8.length) {
      const chunk = Math.min(u8.length - done, 1 << 30);
      done += fs.readSync(this.fd, u8, done, chunk, this.dataStart + a + done);
    }
    return u8;
  }

  async f32(name) {
    const t = this.info(name);
    const u8 = await this.bytes(name);
    if (t.dtype === "F32") return new Float32Array(u8.buffer, u8.byteOffset, u8.byteLength / 4);
    if (t.dtype === "BF16") return bf16ToF32(u8);
    if (t.dtype === "F16") return f16ToF32(u8);
    throw new Error(`${name}: cannot read ${t.dtype} as f32`);
  }

  // bf16 bit patterns of a floating tensor
  async bf16(name) {
    const t = this.info(name);
    if (t.dtype === "BF16") return this.bytes(name);
    const u16 = f32ToBf16(await this.f32(name));
    return new Uint8Array(u16.buffer);
  }

  async quantMeta(base) {
    if (!this.has(base + "comfy_quant")) return null;
    const u8 = await this.bytes(base + "comfy_quant");
    return JSON.parse(Buffer.from(u8).toString("utf8"));
  }

  // Rows `ids` of a 2-D table (embeddings) as fp32, read row by row from the file
  // (app/weights.js:97-108).
  async rows(name, ids) {
    const t = this.info(name);
    const dim = t.shape[1];
    const rowBytes = dim * BYTES[t.dtype];
    const out = new Float32Array(ids.length * dim);
    const u8 = new Uint8Array(rowBytes);
    ids.forEach((id, i) => {
      if (id < 0 || id >= t.shape[0]) throw new Error(`${name}: row ${id} out of range`);
      fs.readSync(this.fd, u8, 0, rowBytes, this.dataStart + t.data_offsets[0] + id * rowBytes);
      const row = t.dtype === "BF16" ? bf16ToF32(u8) : t.dtype === "F16" ? f16ToF32(u8) : new Float32Array(u8.slice().buffer);
      out.set(row, i * dim);
    });
    return out;
  }

  // f32 vector on the GPU; add: a constant added to every element (app/weights.js:111-115)
  async vector(gpu, name, add = 0) {
    const v = await this.f32(name);
    return gpu.upload(add ? v.map((x) => x + add) : v);
  }

  // "<base>weight" (+ optional "<base>bias") as a linear weight object (app/weights.js:117-133)
  async linear(gpu, base) {
    const w = this.info(base + "weight");
    const N = w.shape[0];
    const K = w.shape.slice(1).reduce((a, b) => a * b, 1);
    const bias = this.has(base + "bias") ? await this.vector(gpu, base + "bias") : null;
    const name = base.replace(/\.$/, "");
    const meta = await this.quantMeta(base);
    if (meta) {
      if (meta.format !== "int8_tensorwise" || !meta.convrot) {
        throw new Error(`${base}: unsupported quantization ${JSON.stringify(meta)}`);
      }
      if (w.dtype !== "I8") throw new Error(`${base}weight: expected I8, got ${w.dtype}`);
      const group = meta.convrot_groupsize || 256;
      if (group !== 256 || K % 256) throw new Error(`${base}: ConvRot group ${group} with K=${K} is not supported`);
      return { kind: "i8", N, K, buf: gpu.upload(await this.bytes(base + "weight")), scale: await this.vector(gpu, base + "weight_scale"), bias, name };
    }
    return { kind: "bf16", N, K, buf: gpu.upload(await this.bf16(base + "weight")), bias, name };
  }
}

// Stack bf16 linears that share an input into one [sum N, K] weight (q, k, v -> qkv), with
// `parts` naming each slice; biases are stacked too, zero for parts without one
// (app/weights.js:148-172). The copies run on the device; the parts' buffers are freed.
export function concatLinears(gpu, Ws) {
  const { K } = Ws[0];
  if (!Ws.every((w) => w.kind === "bf16" && w.K === K)) throw new Error("concatLinears: mismatched weights");
  if (K % 2) throw new Error("concatLinears: K must be even");
  const N = Ws.reduce((a, w) => a + w.N, 0);
  const out = { kind: "bf16", K, N, parts: [], bias: null };
  let off = 0;
  for (const w of Ws) {
    out.parts.push({ name: w.name, off, n: w.N });
    off += w.N;
  }
  // bf16 rows as 32-bit words (K even), copied with the elementwise copy op
  out.buf = gpu.upload(new Uint32Array((N * K) / 2));
  off = 0;
  for (const w of Ws) {
    const words = (w.N * K) / 2;
    native.elementwise(EW.copy, addr(w.buf), null, addr(out.buf) + BigInt(off * K * 2), words);
    off += w.N;
  }
  if (Ws.some((w) => w.bias)) {
    out.bias = gpu.upload(new Float32Array(N));
    off = 0;
    for (const w of Ws) {
      if (w.bias) native.elementwise(EW.copy, addr(w.bias), null, addr(out.bias) + BigInt(off * 4), w.N);
      off += w.N;
    }
  }
  native.sync();
  for (const w of Ws) {
    w.buf.destroy();
    if (w.bias) w.bias.destroy();
  }
  return out;
}
