// Weight files for the Node host: a safetensors reader over a local file and the linear weight
// objects the ops take, { kind: "i8" | "bf16", N, K, buf, scale?, bias?, name } (the object
// format of app/weights.js:121-133, so model code and LoRA matching read the same fields).
//
// The reader indexes the header once, checks every entry against the file (known dtype, byte
// range inside the data section, size = product of the shape), and reads tensors with
// positioned reads: nothing is mapped or loaded whole.
//
// int8 layers are ComfyUI's comfy_quant layout written by tools/build_assets.py:35-56:
// `weight` I8 [N, K], `weight_scale` F32 [N, 1] (or [N]) and `comfy_quant` (U8 JSON) with
// format "int8_tensorwise", convrot = true and 256-feature rotation groups. Any other
// quantization is refused, as in app/weights.js:127-129. Every other linear is uploaded as bf16
// bit patterns and decoded in the GEMM.

import fs from "fs";
import { addr } from "./device.js";
import { native, EW } from "./native.js";

const ELEMENT_BYTES = { F64: 8, F32: 4, F16: 2, BF16: 2, I64: 8, I32: 4, I16: 2, I8: 1, U8: 1, BOOL: 1 };
const READ_CHUNK = 1 << 30;

// ---- float formats -------------------------------------------------------------------------

// bf16 -> f32: a bf16 value is the high half of the f32 word. On a little-endian host that half
// is the odd 16-bit slot of each output word; the even slot stays zero.
function widenBf16(u8) {
  const src = new Uint16Array(u8.buffer, u8.byteOffset, u8.byteLength >> 1);
  const out = new Float32Array(src.length);
  const slots = new Uint16Array(out.buffer);
  for (let i = 0; i < src.length; i++) slots[2 * i + 1] = src[i];
  return out;
}

// f16 -> f32 through a table of all 65536 codes, built on first use from the IEEE fields:
// normal codes are (1024 + fraction) * 2^(exponent - 25), subnormal ones fraction * 2^-24.
let f16Codes = null;
function widenF16(u8) {
  if (!f16Codes) {
    f16Codes = new Float32Array(65536);
    for (let code = 0; code < 65536; code++) {
      const exponent = (code >> 10) & 0x1f;
      const fraction = code & 0x3ff;
      let magnitude;
      if (exponent === 0x1f) magnitude = fraction ? NaN : Infinity;
      else if (exponent === 0) magnitude = fraction * 2 ** -24;
      else magnitude = (1024 + fraction) * 2 ** (exponent - 25);
      f16Codes[code] = code & 0x8000 ? -magnitude : magnitude;
    }
  }
  const src = new Uint16Array(u8.buffer, u8.byteOffset, u8.byteLength >> 1);
  const out = new Float32Array(src.length);
  for (let i = 0; i < src.length; i++) out[i] = f16Codes[src[i]];
  return out;
}

// f32 -> bf16 bit patterns: the high 16 bits, rounded half to even on the 16 bits dropped;
// NaNs stay (quiet) NaNs, finite values past the bf16 range round to infinity.
function narrowToBf16(f32) {
  const words = new Uint32Array(f32.buffer, f32.byteOffset, f32.length);
  const out = new Uint16Array(words.length);
  for (let i = 0; i < words.length; i++) {
    const w = words[i];
    const high = w >>> 16;
    const low = w & 0xffff;
    if ((w & 0x7f800000) === 0x7f800000 && (w & 0x7fffff)) out[i] = high | 0x0040;
    else out[i] = low > 0x8000 || (low === 0x8000 && (high & 1)) ? high + 1 : high;
  }
  return out;
}

// Small tensors in other element types (a LoRA alpha saved as an integer or a double).
function widenOther(dtype, u8) {
  const dv = new DataView(u8.buffer, u8.byteOffset, u8.byteLength);
  const n = u8.byteLength / ELEMENT_BYTES[dtype];
  const out = new Float32Array(n);
  const get = {
    F64: (i) => dv.getFloat64(8 * i, true), I64: (i) => Number(dv.getBigInt64(8 * i, true)),
    I32: (i) => dv.getInt32(4 * i, true), I16: (i) => dv.getInt16(2 * i, true),
    I8: (i) => dv.getInt8(i), U8: (i) => dv.getUint8(i), BOOL: (i) => dv.getUint8(i),
  }[dtype];
  for (let i = 0; i < n; i++) out[i] = get(i);
  return out;
}

// ---- the reader ----------------------------------------------------------------------------

export class SafeTensors {
  static async open(path) {
    return new SafeTensors(path);
  }

  constructor(path) {
    this.path = path;
    this.fd = fs.openSync(path, "r");
    const fileBytes = fs.fstatSync(this.fd).size;
    const lenBuf = Buffer.alloc(8);
    if (fs.readSync(this.fd, lenBuf, 0, 8, 0) !== 8) throw new Error(`${path}: not a safetensors file`);
    const headerBytes = Number(lenBuf.readBigUInt64LE(0));
    if (8 + headerBytes > fileBytes) throw new Error(`${path}: header length ${headerBytes} exceeds the file`);
    const text = Buffer.alloc(headerBytes);
    fs.readSync(this.fd, text, 0, headerBytes, 8);
    const header = JSON.parse(text.toString("utf8"));
    this.metadata = header.__metadata__ || {};
    const dataStart = 8 + headerBytes;
    const dataBytes = fileBytes - dataStart;
    this.entries = new Map();
    for (const [name, e] of Object.entries(header)) {
      if (name === "__metadata__") continue;
      const size = ELEMENT_BYTES[e.dtype];
      if (!size) throw new Error(`${path}: ${name} has unsupported dtype ${e.dtype}`);
      const [begin, end] = e.data_offsets;
      const count = e.shape.reduce((a, b) => a * b, 1);
      if (!(begin >= 0 && end <= dataBytes && end - begin === count * size)) {
        throw new Error(`${path}: ${name} [${e.shape}] ${e.dtype} does not match its byte range [${begin}, ${end})`);
      }
      this.entries.set(name, { dtype: e.dtype, shape: e.shape, pos: dataStart + begin, bytes: end - begin });
    }
  }

  close() {
    if (this.fd !== null) fs.closeSync(this.fd);
    this.fd = null;
  }

  names() {
    return [...this.entries.keys()];
  }

  has(name) {
    return this.entries.has(name);
  }

  // { dtype, shape } of a tensor
  info(name) {
    const e = this.entries.get(name);
    if (!e) throw new Error(`${this.path}: no tensor ${name}`);
    return e;
  }

  // Positioned read of `bytes` bytes at file position `pos` into a fresh buffer.
  readAt(pos, bytes) {
    const u8 = new Uint8Array(new ArrayBuffer(bytes));
    for (let done = 0; done < bytes;) {
      const got = fs.readSync(this.fd, u8, done, Math.min(bytes - done, READ_CHUNK), pos + done);
      if (got <= 0) throw new Error(`${this.path}: short read at ${pos + done}`);
      done += got;
    }
    return u8;
  }

  // The stored bytes of a tensor.
  async bytes(name) {
    const e = this.info(name);
    return this.readAt(e.pos, e.bytes);
  }

  // A tensor's values as f32, whatever its element type.
  async f32(name) {
    const e = this.info(name);
    return this.decode(e.dtype, await this.bytes(name));
  }

  decode(dtype, u8) {
    if (dtype === "F32") return new Float32Array(u8.buffer, u8.byteOffset, u8.byteLength >> 2);
    if (dtype === "BF16") return widenBf16(u8);
    if (dtype === "F16") return widenF16(u8);
    return widenOther(dtype, u8);
  }

  // A floating tensor as bf16 bit patterns (bytes).
  async bf16(name) {
    const e = this.info(name);
    if (e.dtype === "BF16") return this.bytes(name);
    return new Uint8Array(narrowToBf16(await this.f32(name)).buffer);
  }

  // Rows `ids` of a 2-D table (embeddings) as f32 [ids.length, dim], without reading the table
  // whole: the distinct ids are sorted and each run of consecutive rows is one read
  // (app/weights.js:97-108 reads row by row).
  async rows(name, ids) {
    const e = this.info(name);
    const [count, dim] = e.shape;
    const rowBytes = dim * ELEMENT_BYTES[e.dtype];
    for (const id of ids) if (!(id >= 0 && id < count)) throw new Error(`${name}: row ${id} is outside [0, ${count})`);
    const sorted = [...new Set(ids)].sort((a, b) => a - b);
    const found = new Map();
    for (let i = 0; i < sorted.length;) {
      let j = i + 1;
      while (j < sorted.length && sorted[j] === sorted[j - 1] + 1) j++;
      const run = this.decode(e.dtype, this.readAt(e.pos + sorted[i] * rowBytes, (j - i) * rowBytes));
      for (let r = i; r < j; r++) found.set(sorted[r], run.subarray((r - i) * dim, (r - i + 1) * dim));
      i = j;
    }
    const out = new Float32Array(ids.length * dim);
    ids.forEach((id, i) => out.set(found.get(id), i * dim));
    return out;
  }

  // f32 vector on the GPU; add: a constant added to every element (Gemma3 stores its norm
  // weights as w - 1, app/weights.js:111-115)
  async vector(gpu, name, add = 0) {
    const v = await this.f32(name);
    if (add) for (let i = 0; i < v.length; i++) v[i] += add;
    return gpu.upload(v);
  }

  // The comfy_quant JSON of a layer, or null for an unquantized one.
  async quantization(base) {
    if (!this.has(base + "comfy_quant")) return null;
    return JSON.parse(Buffer.from(await this.bytes(base + "comfy_quant")).toString("utf8"));
  }

  // "<base>weight" (+ "<base>bias") as a linear weight object; weights with more than two
  // dimensions are flattened to [N, K] (app/weights.js:117-133).
  async linear(gpu, base) {
    const weight = base + "weight";
    const w = this.info(weight);
    const N = w.shape[0];
    const K = w.shape.slice(1).reduce((a, b) => a * b, 1);
    const layer = { kind: "bf16", N, K, name: base.endsWith(".") ? base.slice(0, -1) : base, bias: null };
    const quant = await this.quantization(base);
    if (quant) {
      if (quant.format !== "int8_tensorwise" || !quant.convrot) {
        throw new Error(`${base}: unsupported quantization ${JSON.stringify(quant)}`);
      }
      if (w.dtype !== "I8") throw new Error(`${weight}: an int8_tensorwise weight must be I8, not ${w.dtype}`);
      const group = quant.convrot_groupsize === undefined ? 256 : quant.convrot_groupsize;
      if (group !== 256 || K % 256) throw new Error(`${base}: ConvRot groups of ${group} over K=${K} are not supported`);
      const s = this.info(base + "weight_scale");
      if (s.shape.reduce((a, b) => a * b, 1) !== N) throw new Error(`${base}weight_scale [${s.shape}] is not one scale per row of ${N}`);
      layer.kind = "i8";
      layer.buf = gpu.upload(await this.bytes(weight));
      layer.scale = await this.vector(gpu, base + "weight_scale");
    } else {
      layer.buf = gpu.upload(await this.bf16(weight));
    }
    if (this.has(base + "bias")) layer.bias = await this.vector(gpu, base + "bias");
    return layer;
  }
}

// Stack linears that share an input into one [sum N, K] weight (q, k, v -> qkv; the DiT's kv_y
// projections of every joint block), with `parts` naming each slice; per-row scales (int8) and
// biases are stacked too, zero bias for parts without one (app/weights.js:148-172). All parts
// are bf16, or all int8 ConvRot. The copies run on the device; the parts' buffers are freed.
export function concatLinears(gpu, Ws) {
  const { K, kind } = Ws[0];
  if (!Ws.every((w) => w.kind === kind && w.K === K && (kind === "bf16" || kind === "i8"))) {
    throw new Error("concatLinears: the weights must share K and be all bf16 or all int8");
  }
  const rowBytes = kind === "i8" ? K : 2 * K;
  if (rowBytes % 4) throw new Error("concatLinears: rows must be whole 32-bit words");
  const N = Ws.reduce((a, w) => a + w.N, 0);
  const name = Ws.length > 2 ? `${Ws[0].name} + ... + ${Ws[Ws.length - 1].name}` : Ws.map((w) => w.name).join(" + ");
  const out = { name, kind, K, N, parts: [], bias: null };
  let off = 0;
  for (const w of Ws) {
    out.parts.push({ name: w.name, off, n: w.N });
    off += w.N;
  }
  // rows as 32-bit words, copied with the elementwise copy op; f32 vectors likewise
  const stack = (field, bytesPerRow) => {
    const dst = gpu.upload(new Uint32Array((N * bytesPerRow) / 4));
    let r = 0;
    for (const w of Ws) {
      if (w[field]) native.elementwise(EW.copy, addr(w[field]), null, addr(dst) + BigInt(r * bytesPerRow), (w.N * bytesPerRow) / 4);
      r += w.N;
    }
    return dst;
  };
  out.buf = stack("buf", rowBytes);
  if (kind === "i8") out.scale = stack("scale", 4);
  if (Ws.some((w) => w.bias)) out.bias = stack("bias", 4);
  native.sync();
  for (const w of Ws) {
    w.buf.destroy();
    if (w.scale) w.scale.destroy();
    if (w.bias) w.bias.destroy();
  }
  return out;
}
