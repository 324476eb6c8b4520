// Tensor ops with the call surface of the reference's app/gpu/ops.js, launched as HIP kernels
// through the ns2 addon. Activations are fp32 Tensors (row-major); offsets and strides are in
// elements. Three fused producers are added for the int8 layers: normModRotated,
// gluRotated and rotateHalf write the rotated fp16 operand that linear() takes as opts.xr,
// so the separate rotation pass of the reference never runs on the DiT path. With
// tiled = true they write it in the tiled layout of the fast int8 GEMM (rows padded to a
// multiple of 64), which linear() then multiplies with the weight re-tiled by tileWeight().

import { addr, DeviceBuffer } from "./device.js";
import { native, ACT, EW } from "./native.js";
import { loraArgs, loraLaunches } from "./lora.js";

const opt = (v, d) => (v === undefined || v === null ? d : v);

// int8 weights are ConvRot-quantized: they take Hadamard-rotated inputs (app/gpu/ops.js:34-35)
export const needsRotation = (W) => W.kind === "i8";

// ConvRot input rotation, fp32 -> fp32 (app/gpu/ops.js:37-44).
export function rotate(gpu, x) {
  const y = gpu.empty(x.shape);
  const groups = x.size / 256;
  gpu.run("hadamard", 0, () => native.hadamard256(addr(x), addr(y), groups));
  return y;
}

// fp16 GEMM operand [rows, cols]: row-major, or tiled (tile images of 64 rows x 64 columns,
// rows padded to a multiple of 64; y.rows keeps the real count).
function rotatedOperand(gpu, rows, cols, tiled) {
  const y = gpu.empty([tiled ? Math.ceil(rows / 64) * 64 : rows, cols], "f16");
  if (tiled) {
    y.tiled = true;
    y.rows = rows;
  }
  return y;
}

// Rotation written as the fp16 GEMM operand ([rows, cols], cols % 256 == 0).
export function rotateHalf(gpu, x, cols = x.shape[x.shape.length - 1], tiled = false) {
  const rows = x.size / cols;
  const y = rotatedOperand(gpu, rows, cols, tiled);
  gpu.run("rotate_f16", 0, () => native.rotateF16(addr(x), cols, addr(y), cols, rows, cols, tiled ? 1 : 0));
  return y;
}

// Whether an int8 weight can take tiled (rotated) operands (N % 64 == 0, K % 256 == 0).
export const tileable = (W) => W.kind === "i8" && W.N % 64 === 0 && W.K % 256 === 0;
// Whether a bf16 weight can be re-tiled as fp16 for tiled plain operands (N, K % 64 == 0).
export const tileablePlain = (W) => W.kind === "bf16" && W.N % 64 === 0 && W.K % 64 === 0;

// Re-tile a weight for tiled operands (W.tbuf, kept next to the row-major W.buf): int8 tiles of
// biased bytes, or fp16 tiles of a bf16 weight.
export function tileWeight(gpu, W) {
  if (!tileable(W) && !tileablePlain(W)) throw new Error(`${W.name}: [${W.N}, ${W.K}] ${W.kind} weight cannot be tiled`);
  if (W.tbuf) return W;
  const bytes = W.N * W.K * (W.kind === "i8" ? 1 : 2);
  W.tbuf = new DeviceBuffer(native.malloc(bytes), bytes, false);
  if (W.kind === "i8") gpu.run("tile_i8_weight", 0, () => native.tileI8Weight(addr(W.buf), addr(W.tbuf), W.N, W.K));
  else gpu.run("tile_bf16_weight", 0, () => native.tileBf16Weight(addr(W.buf), addr(W.tbuf), W.N, W.K));
  return W;
}

// x (- sub) as the tiled fp16 operand of a linear over a re-tiled bf16 weight ([rows, cols],
// cols % 64 == 0): the DiT's patch-embedder input, and the SPRINT projection's input g - x
// (app/models/nanosaur2.js:236-243: elementwise sub, then linear) without the fp32 difference.
export function toTiled(gpu, x, sub = null) {
  const cols = x.shape[x.shape.length - 1];
  const rows = x.size / cols;
  const y = rotatedOperand(gpu, rows, cols, true);
  gpu.run(sub ? "sub_tiled_f16" : "to_tiled_f16", 0, () =>
    native.toTiledF16(addr(x), cols, sub ? addr(sub) : null, cols, addr(y), rows, cols));
  return y;
}

// normMod (below) written as the tiled fp16 operand of a linear over a re-tiled bf16 weight
// (the final layer, app/models/nanosaur2.js:252-253), cols % 256 == 0.
export function normModTiled(gpu, x, mod, shiftOff, scaleOff, cols, weight = null, eps = 1e-6) {
  const rows = x.size / cols;
  const y = rotatedOperand(gpu, rows, cols, true);
  gpu.run(weight ? "rmsnorm_mod_f16" : "layernorm_mod_f16", 0, () =>
    native.normModF16(addr(x), addr(mod), shiftOff, scaleOff, rows, cols, addr(weight), eps, addr(y), 1));
  return y;
}

// Free the row-major int8 copy of a re-tiled weight when the caller only ever feeds it tiled
// operands (the fused DiT path): the tiled copy alone then holds the weight, so the int8
// model stays resident once instead of twice. linear() refuses a row-major launch afterwards.
export function dropRowMajor(W) {
  if (!W.tbuf && !W.tglu) throw new Error(`${W.name}: only a re-tiled weight can drop its row-major copy`);
  if (W.buf) W.buf.destroy();
  W.buf = null;
  return W;
}

// Re-tile the GLU MLP's first int8 weight [2I, K] with its two halves interleaved (W.tglu),
// for linearGluRotated.
export function tileWeightGlu(gpu, W) {
  if (W.kind !== "i8" || W.N % 512 !== 0 || W.K % 256 !== 0) throw new Error(`${W.name}: [${W.N}, ${W.K}] cannot take the fused GLU path`);
  if (W.tglu) return W;
  const ptr = native.malloc(W.N * W.K);
  W.tglu = new DeviceBuffer(ptr, W.N * W.K, false);
  gpu.run("tile_i8_weight", 0, () => native.tileI8WeightGlu(addr(W.buf), addr(W.tglu), W.N, W.K));
  return W;
}

// glu(linear(x, W), act) rotated, as the tiled fp16 operand of the next int8 linear: one
// kernel for ops.linear + ops.glu + ops.rotate of the MLP (app/gpu/ops.js:46-66, 140-148,
// 37-44). xr is a tiled operand (normModRotated(..., tiled = true)).
export function linearGluRotated(gpu, xr, W, act, name = "gemm.i8.glu") {
  if (!xr.tiled || !W.tglu) throw new Error(`${W.name}: linearGluRotated needs a tiled operand and tileWeightGlu`);
  const M = xr.rows, I = W.N / 2;
  const y = rotatedOperand(gpu, M, I, true);
  const lora = loraArgs(gpu, W);
  gpu.run(name, 2 * M * W.N * W.K, () =>
    native.linearI8GluRotTiled(addr(xr), addr(W.tglu), addr(W.scale), addr(W.bias || null), addr(y), M, W.N, W.K, 1,
      ACT[act], ...lora));
  return y;
}

// The attention's packed fp16 values for Lk keys of H heads of D (filled by linear() with
// opts.vpack, read by attention() with opts.vPacked).
export function packedValues(gpu, Lk, H, D) {
  const halfs = native.attentionVpackBytes(Lk, H, D) / 2;
  const t = gpu.empty([halfs], "f16");
  t.vpack = { Lk, H, D };
  return t;
}

// y = x @ W^T (+ bias) (act) (app/gpu/ops.js:46-66). opts: out, resid, gate, gOff, ldc, cOff,
// bias, act, xr (pre-rotated input of an int8 weight: fp32 from rotate() or fp16 from a fused
// producer), name. x may be null when xr is given. opts.vpack = { buf, col0 } (tiled int8 only,
// no resid): the output columns from col0 on (the last H*D) are written into buf, a
// packedValues() tensor, as the values of keys [0, M), instead of into out.
export function linear(gpu, x, W, opts = {}) {
  const src = opts.xr || x;
  const M = src.tiled ? src.rows : src.size / W.K;
  const out = opts.out || gpu.empty([M, W.N]);
  const ldc = opt(opts.ldc, W.N);
  const cOff = opt(opts.cOff, 0);
  const gOff = opt(opts.gOff, 0);
  const bias = opts.bias || W.bias || null;
  const act = ACT[opts.act || "none"];
  if (act === undefined) throw new Error(`linear: unknown activation ${opts.act}`);
  const resid = opts.resid ? 1 : 0;
  if (W.kind === "i8" && src.tiled && opts.vpack) {
    if (!W.tbuf) throw new Error(`${W.name}: a tiled operand needs the tiled weight (tileWeight)`);
    if (resid) throw new Error("linear: packed values take a plain store (no resid)");
    const lora = loraArgs(gpu, W);
    const { buf, col0 } = opts.vpack;
    const { Lk, H, D } = buf.vpack;
    gpu.run(opts.name || "gemm.i8", 2 * M * W.N * W.K, () =>
      native.linearI8TiledVpack(addr(src), addr(W.tbuf), addr(W.scale), addr(bias), addr(out), M, W.N, W.K, ldc,
        cOff, 1, act, ...lora, addr(buf), col0, H, D, Lk));
    return out;
  }
  if (src.tiled && !W.tbuf) throw new Error(`${W.name}: a tiled operand needs the tiled weight (tileWeight)`);
  if (W.kind === "i8" && !src.tiled && !W.buf) {
    throw new Error(`${W.name}: the row-major int8 weight was freed after tiling; pass a tiled operand`);
  }
  if (W.kind !== "i8" && W.kind !== "bf16") throw new Error(`linear: weight kind ${W.kind} is not part of this build`);
  // LoRA side paths (W.lora, attached by lora.js): the stacked low-rank term starts the GEMM's
  // accumulators; the down-projection takes the same (rotated) input (app/gpu/ops.js:54-58). A
  // stacked weight whose LoRAs need several side paths launches once per row window of W,
  // each into its own output columns.
  for (const { off, n, args: lora } of loraLaunches(gpu, W)) {
    if (src.tiled && off % 64) throw new Error(`${W.name}: LoRA window at row ${off} is not tile aligned`);
    const rowBytes = W.kind === "i8" ? W.K : 2 * W.K;
    const wAt = (buf) => addr(buf) + BigInt(off * rowBytes);
    const vAt = (t) => (t ? addr(t) + BigInt(4 * off) : null);
    const flops = 2 * M * n * W.K;
    const c0 = cOff + off, g0 = gOff + off;
    if (W.kind === "i8" && src.tiled) {
      gpu.run(opts.name || "gemm.i8", flops, () =>
        native.linearI8Tiled(addr(src), wAt(W.tbuf), vAt(W.scale), vAt(bias), addr(out), M, n, W.K, ldc,
          c0, 1, act, resid, addr(opts.gate), g0, ...lora));
    } else if (W.kind === "i8") {
      const aFmt = opts.xr ? (opts.xr.dtype === "f16" ? 1 : 2) : 0;
      gpu.run(opts.name || "gemm.i8", flops, () =>
        native.linearI8(addr(src), aFmt, W.K, wAt(W.buf), vAt(W.scale), vAt(bias), null, addr(out),
          M, n, W.K, ldc, c0, 1, act, resid, addr(opts.gate), g0, ...lora));
    } else if (src.tiled) {
      gpu.run(opts.name || "gemm.bf16", flops, () =>
        native.linearF16wTiled(addr(src), wAt(W.tbuf), vAt(bias), addr(out), M, n, W.K, ldc, c0, 1, act, resid,
          addr(opts.gate), g0, ...lora));
    } else {
      if (!W.buf) throw new Error(`${W.name}: the row-major bf16 weight was freed after tiling; pass a tiled operand`);
      gpu.run(opts.name || "gemm.bf16", flops, () =>
        native.linearBf16(addr(x), W.K, wAt(W.buf), vAt(bias), null, addr(out), M, n, W.K, ldc, c0,
          1, act, resid, addr(opts.gate), g0, ...lora));
    }
  }
  return out;
}

export function zero(gpu, t) {
  const words = t.dtype === "f16" ? Math.ceil(t.size / 2) : t.size;
  gpu.run("zero", 0, () => native.fill(addr(t), 0, words));
}

export function rmsnorm(gpu, x, weight, cols, eps = 1e-6, out) {
  const rows = x.size / cols;
  const y = out || gpu.empty(x.shape);
  gpu.run("rmsnorm", 0, () => native.rmsnorm(addr(x), addr(weight), addr(y), rows, cols, eps));
  return y;
}

// [rows, cols] -> [cols, rows] (the latent <-> token layout change of the reference's forward,
// app/models/nanosaur2.js:220-221, 254-255, on the device; addition to the reference ops).
export function transpose(gpu, x) {
  const [rows, cols] = x.shape;
  const y = gpu.empty([cols, rows]);
  gpu.run("transpose", 0, () => native.transpose(addr(x), addr(y), rows, cols));
  return y;
}

// x += rmsnorm(a) * wAdd; returns rmsnorm(x) * wOut (or null without wOut): a sandwich norm,
// its residual add and the following norm in one launch (app/models/gemma3.js:76-80, 87-88;
// addition to the reference ops).
export function addRmsnorm(gpu, x, a, wAdd, wOut, cols, eps = 1e-6) {
  const rows = x.size / cols;
  const y = wOut ? gpu.empty(x.shape) : null;
  gpu.run("add_rmsnorm", 0, () => native.addRmsnorm(addr(x), addr(a), addr(wAdd), addr(wOut), addr(y), rows, cols, eps));
  return y;
}

// linear(a, W) followed by glu(., act) for a bf16 gate/up weight without LoRA: the split-K sums
// feed the GLU directly, so the [M, 2I] product never reaches HBM (app/models/gemma3.js:79-82;
// addition to the reference ops). Other weights take the two ops.
export function linearGlu(gpu, a, W, act) {
  if (W.kind !== "bf16" || (W.lora && W.lora.length)) {
    const t = linear(gpu, a, W, { name: "te.mlp" });
    const y = glu(gpu, t, act);
    t.release();
    return y;
  }
  if (ACT[act] === undefined) throw new Error(`linearGlu: unknown activation ${act}`);
  const M = a.size / W.K;
  const y = gpu.empty([M, W.N / 2]);
  gpu.run("te.mlp+glu", 2 * M * W.N * W.K, () =>
    native.linearBf16Glu(addr(a), W.K, addr(W.buf), addr(W.bias || null), addr(y), M, W.N, W.K, ACT[act]));
  return y;
}

// linear(a, W) of a stacked q|k|v weight followed by headNorm2 on its q and k heads (Gemma3,
// app/models/gemma3.js:62-67; addition to the reference ops): for a bf16 weight without LoRA the
// split-K sums are normed (and rotated) in the same row kernel, else the two ops run.
// f16kv: on the fused path, heads from H1 on (keys and values) are written as fp16 into the
// front half of their own fp32 columns (fp16 column 2*H1*D + j of each row, row stride 2*W.N fp16
// elements), and the result carries .f16kv = { off, ld } in fp16 elements for
// attentionRowsF16kv; the fp32 columns of those heads are then not written.
export function linearHeadNorm(gpu, a, W, w1, H1, w2, H2, { D, cs = null, eps = 1e-6, f16kv = false }) {
  const M = a.size / W.K;
  if (W.kind !== "bf16" || (W.lora && W.lora.length)) {
    const t = linear(gpu, a, W, { name: "te.qkv" });
    headNorm2(gpu, t, w1, H1, w2, H2, { L: M, D, ld: W.N, cs, eps });
    return t;
  }
  const y = gpu.empty([M, W.N]);
  if (f16kv) {
    const kv16 = addr(y) + BigInt(H1 * D * 4);
    gpu.run("te.qkv+head_norm", 2 * M * W.N * W.K, () =>
      native.linearBf16HeadNormF16kv(addr(a), W.K, addr(W.buf), addr(W.bias || null), addr(y), M, W.N, W.K,
        addr(w1), H1, addr(w2), H2, D, cs ? addr(cs) : null, cs ? cs.sinOff : 0, cs ? M : 0, eps, kv16, 2 * W.N));
    y.f16kv = { off: 2 * H1 * D, ld: 2 * W.N };
    return y;
  }
  gpu.run("te.qkv+head_norm", 2 * M * W.N * W.K, () =>
    native.linearBf16HeadNorm(addr(a), W.K, addr(W.buf), addr(W.bias || null), addr(y), M, W.N, W.K, addr(w1), H1,
      addr(w2), H2, D, cs ? addr(cs) : null, cs ? cs.sinOff : 0, cs ? M : 0, eps));
  return y;
}

// attentionRowsF16kv and the output projection after it (a Gemma3 layer's attention and o_proj,
// app/models/gemma3.js:67-73; addition to the reference ops) without the attention output in
// HBM: each head's block multiplies its normalized output by its D columns of W_o (a bf16 weight
// re-tiled as fp16, W.tbuf) into its share part[h] [Lq, W.N]; the H shares sum to the projection
// without bias (partsAddRmsnorm adds them and the bias). Returns the shares [H, Lq, W.N].
export function attentionRowsF16kvOproj(gpu, { q, kv, Lq, Lk, H, D, ldq, qOff = 0, kOff, vOff, ldkv, group = 1,
  causal = false, W }) {
  if (!W.tbuf || W.kind !== "bf16" || W.K !== H * D) throw new Error(`${W.name}: the fused projection needs a re-tiled bf16 weight of K = H*D`);
  const part = gpu.empty([H, Lq, W.N]);
  gpu.run("attn.rows+o", 4 * Lq * Lk * D * H + 2 * Lq * W.N * W.K, () =>
    native.attentionRowsF16kvOproj(addr(q), addr(kv), addr(kv), addr(W.tbuf), addr(part), Lq, Lk, H, D, ldq, ldkv,
      ldkv, qOff, kOff, vOff, group, causal ? 1 : 0, W.N));
  return part;
}

// GLU output columns per share of linearGluDown (the library's group width)
export const GLU_DOWN_GROUP = 128;

// linearGlu(a, W) and the linear by Wd after it (Gemma3's gate/up, GLU and down projection,
// app/models/gemma3.js:79-83; addition to the reference ops) without the GLU output in HBM: the
// GLU's row kernel multiplies each 128-column group of its output by Wd's matching columns
// (a bf16 weight re-tiled as fp16, Wd.tbuf). Returns the shares [W.N/256, M, Wd.N]; they sum
// to the product without bias (partsAddRmsnorm adds them and the bias).
export function linearGluDown(gpu, a, W, Wd, act = "gelu_tanh") {
  if (!Wd.tbuf || Wd.kind !== "bf16" || Wd.K !== W.N / 2) throw new Error(`${Wd.name}: the fused down projection needs a re-tiled bf16 weight of K = N/2`);
  const M = a.size / W.K;
  const part = gpu.empty([W.N / (2 * GLU_DOWN_GROUP), M, Wd.N]);
  gpu.run("te.mlp+glu+down", 2 * M * W.N * W.K + 2 * M * Wd.N * Wd.K, () =>
    native.linearBf16GluDown(addr(a), W.K, addr(W.buf), addr(W.bias || null), M, W.N, W.K, ACT[act], addr(Wd.tbuf),
      Wd.N, addr(part)));
  return part;
}

// Whether a bf16 weight takes the encoder's tiled fp16 path (re-tiled, no LoRA attached).
export const tiledPathOk = (W) => W.kind === "bf16" && !!W.tbuf && !(W.lora && W.lora.length);

// linearHeadNorm with f16kv on a tiled fp16 operand (aT, rows aT.rows) over W.tbuf: the same
// result and .f16kv layout.
export function linearHeadNormTiled(gpu, aT, W, w1, H1, w2, H2, { D, cs = null, eps = 1e-6 }) {
  const M = aT.rows;
  const y = gpu.empty([M, W.N]);
  const kv16 = addr(y) + BigInt(H1 * D * 4);
  gpu.run("te.qkv+head_norm", 2 * M * W.N * W.K, () =>
    native.linearF16wTiledHeadNormF16kv(addr(aT), addr(W.tbuf), addr(W.bias || null), addr(y), M, W.N, W.K,
      addr(w1), H1, addr(w2), H2, D, cs ? addr(cs) : null, cs ? cs.sinOff : 0, cs ? M : 0, eps, kv16, 2 * W.N));
  y.f16kv = { off: 2 * H1 * D, ld: 2 * W.N };
  return y;
}

// linearGluDown on a tiled fp16 operand (aT, rows aT.rows) with W.tbuf: the same shares.
export function linearGluDownTiled(gpu, aT, W, Wd, act = "gelu_tanh") {
  if (!Wd.tbuf || Wd.kind !== "bf16" || Wd.K !== W.N / 2) throw new Error(`${Wd.name}: the fused down projection needs a re-tiled bf16 weight of K = N/2`);
  const M = aT.rows;
  const part = gpu.empty([W.N / (2 * GLU_DOWN_GROUP), M, Wd.N]);
  gpu.run("te.mlp+glu+down", 2 * M * W.N * W.K + 2 * M * Wd.N * Wd.K, () =>
    native.linearF16wTiledGluDown(addr(aT), addr(W.tbuf), addr(W.bias || null), M, W.N, W.K, ACT[act],
      addr(Wd.tbuf), Wd.N, addr(part)));
  return part;
}

// partsAddRmsnorm with y written as the tiled fp16 operand of the next linear (returned).
export function partsAddRmsnormTiled(gpu, part, splits, bias, x, wAdd, wOut, eps = 1e-6) {
  const N = x.shape[x.shape.length - 1], M = x.size / N;
  const yt = rotatedOperand(gpu, M, N, true);
  gpu.run("te.proj_norm", 0, () =>
    native.partsAddRmsnormTiled(addr(part), splits, addr(bias || null), addr(x), addr(wAdd), addr(wOut), addr(yt), M,
      N, eps));
  return yt;
}

// addRmsnorm on a product given as `splits` shares [splits, M, N] (+ bias): x += rmsnorm(sum) *
// wAdd, then y = rmsnorm(x) * wOut when wOut is given (returned).
export function partsAddRmsnorm(gpu, part, splits, bias, x, wAdd, wOut, eps = 1e-6) {
  const N = x.shape[x.shape.length - 1], M = x.size / N;
  const y = wOut ? gpu.empty(x.shape) : null;
  gpu.run("te.proj_norm", 0, () =>
    native.partsAddRmsnorm(addr(part), splits, addr(bias || null), addr(x), addr(wAdd), addr(wOut), addr(y), M, N, eps));
  return y;
}

// The materialized-path attention (causal / grouped, as attention() runs it) on fp16 keys and
// values: kv is a Tensor whose bytes hold them, kOff / vOff / ldkv in fp16 elements (the
// .f16kv layout of linearHeadNorm); q fp32 as in attention(). Output [Lq, H*D].
export function attentionRowsF16kv(gpu, { q, kv, Lq, Lk, H, D, ldq, qOff = 0, kOff, vOff, ldkv, group = 1,
  causal = false, out }) {
  const o = out || gpu.empty([Lq, H * D]);
  gpu.run("attn.rows", 4 * Lq * Lk * D * H, () =>
    native.attentionRowsF16kv(addr(q), addr(kv), addr(kv), addr(o), Lq, Lk, H, D, ldq, ldkv, ldkv, H * D, qOff, kOff,
      vOff, group, causal ? 1 : 0));
  return o;
}

// linear(a, W) followed by addRmsnorm(x, ., wAdd, wOut) for a bf16 weight without LoRA: the
// projection's rows are summed and normed in one row kernel, so the [M, N] product never
// reaches HBM (app/models/gemma3.js:72-80, 83-92; addition to the reference ops). Other weights
// take the two ops.
export function linearAddRmsnorm(gpu, a, W, x, wAdd, wOut, eps = 1e-6) {
  if (W.kind !== "bf16" || (W.lora && W.lora.length) || W.N > 1024) {
    const t = linear(gpu, a, W, { name: "te.proj" });
    const y = addRmsnorm(gpu, x, t, wAdd, wOut, W.N, eps);
    t.release();
    return y;
  }
  const M = a.size / W.K;
  const y = wOut ? gpu.empty(x.shape) : null;
  gpu.run("te.proj+norm", 2 * M * W.N * W.K, () =>
    native.linearBf16AddRmsnorm(addr(a), W.K, addr(W.buf), addr(W.bias || null), addr(x), addr(wAdd), addr(wOut),
                                addr(y), M, W.N, W.K, eps));
  return y;
}

// norm(x) * (1 + mod[scaleOff..]) + mod[shiftOff..]; RMSNorm*weight, or LayerNorm without
// affine when weight is null (app/gpu/ops.js:119-129).
export function normMod(gpu, x, mod, shiftOff, scaleOff, cols, weight = null, eps = 1e-6) {
  const rows = x.size / cols;
  const y = gpu.empty(x.shape);
  gpu.run(weight ? "rmsnorm_mod" : "layernorm_mod", 0, () =>
    native.normMod(addr(x), addr(mod), shiftOff, scaleOff, rows, cols, addr(weight), eps, addr(y)));
  return y;
}

// normMod followed by the ConvRot rotation, as the fp16 operand of an int8 linear.
export function normModRotated(gpu, x, mod, shiftOff, scaleOff, cols, weight = null, eps = 1e-6, tiled = false) {
  const rows = x.size / cols;
  const y = rotatedOperand(gpu, rows, cols, tiled);
  gpu.run(weight ? "rmsnorm_mod_rot" : "layernorm_mod_rot", 0, () =>
    native.normModRotateF16(addr(x), addr(mod), shiftOff, scaleOff, rows, cols, addr(weight), eps, addr(y),
      tiled ? 1 : 0));
  return y;
}

// In-place per-head RMSNorm (+ RoPE with a table from common.js) on L rows x H heads of D
// values at X[(rowOff + l) * ld + colOff + h * D] (app/gpu/ops.js:131-138).
export function headNorm(gpu, X, weight, { L, H, D, ld, colOff = 0, rowOff = 0, cs = null, eps = 1e-6 }) {
  gpu.run(cs ? "head_norm_rope" : "head_norm", 0, () =>
    native.headNorm(addr(X), addr(weight), L, H, D, ld, colOff, rowOff, cs ? addr(cs) : null, cs ? cs.sinOff : 0, eps));
}

// headNorm on two adjacent head ranges in one launch: H1 heads with w1 from colOff on, then H2
// heads with w2 (Gemma3's q and k norms; addition to the reference ops).
export function headNorm2(gpu, X, w1, H1, w2, H2, { L, D, ld, colOff = 0, rowOff = 0, cs = null, eps = 1e-6 }) {
  gpu.run(cs ? "head_norm_rope" : "head_norm", 0, () =>
    native.headNorm2(addr(X), addr(w1), H1, addr(w2), H2, L, D, ld, colOff, rowOff, cs ? addr(cs) : null,
                     cs ? cs.sinOff : 0, eps));
}

// [rows, 2I] -> [rows, I]: act(first half) * second half (app/gpu/ops.js:140-148)
export function glu(gpu, x, act) {
  const I = x.shape[1] / 2;
  const y = gpu.empty([x.shape[0], I]);
  gpu.run("glu." + act, 0, () => native.glu(addr(x), addr(y), x.shape[0], I, ACT[act]));
  return y;
}

// glu followed by the ConvRot rotation, as the fp16 operand of an int8 linear.
export function gluRotated(gpu, x, act, tiled = false) {
  const I = x.shape[1] / 2;
  const y = rotatedOperand(gpu, x.shape[0], I, tiled);
  gpu.run("glu_rot." + act, 0, () => native.gluRotateF16(addr(x), addr(y), x.shape[0], I, ACT[act], tiled ? 1 : 0));
  return y;
}

// [1, N] = scale * sum_r w[r] * x[r] (app/gpu/ops.js:150-156)
// y[r, :] = a + b[r, :] for every row of b: the DiT's per-block modulation add
// (app/models/nanosaur2.js:190) for all blocks in one launch (addition to the reference ops).
export function addRows(gpu, a, b) {
  const [rows, n] = b.shape;
  if (a.size !== n) throw new Error(`addRows: a has ${a.size} values, rows have ${n}`);
  const y = gpu.empty([rows, n]);
  gpu.run("add_rows", 0, () => native.addRows(addr(a), addr(b), addr(y), rows, n));
  return y;
}

// Row r of a [rows, n] tensor as a [1, n] view (no copy; valid while t is).
export function rowView(t, r) {
  const n = t.shape[t.shape.length - 1];
  return { buf: { ptr: addr(t) + BigInt(r * n * 4) }, shape: [1, n], size: n, release() {} };
}

// Columns [off, off + n) of a [1, N] tensor as a [1, n] view (no copy; valid while t is).
export function colView(t, off, n) {
  if (t.size !== t.shape[t.shape.length - 1] || off + n > t.size) throw new Error("colView: a [1, N] tensor and a window inside it");
  return { buf: { ptr: addr(t) + BigInt(off * 4) }, shape: [1, n], size: n, release() {} };
}

export function rowSum(gpu, x, w, scale = 1) {
  const [rows, N] = x.shape;
  const y = gpu.empty([1, N]);
  gpu.run("rowsum", 0, () => native.rowSum(addr(x), addr(w), addr(y), rows, N, scale));
  return y;
}

export function elementwise(gpu, op, a, b, out) {
  const y = out || gpu.empty(a.shape);
  if (EW[op] === undefined) throw new Error(`elementwise: unknown op ${op}`);
  gpu.run("elementwise." + op, 0, () => native.elementwise(EW[op], addr(a), b ? addr(b) : null, addr(y), y.size));
  return y;
}

// y += a (in place) (app/gpu/ops.js:187-192)
export function accumulate(gpu, y, a) {
  gpu.run("accumulate", 0, () => native.accumulate(addr(y), addr(a), y.size));
}

// Multi-head attention (app/gpu/ops.js:194-242): the fused flash kernel when non-causal, group
// 1, D % 32 = 0, D <= 128 and 4-aligned; otherwise the materialized path's semantics (causal
// masking, K/V head h / group) on the row kernel.
//  q: [Lq, ldq] with head h at column qOff + h*D; k, v: [Lk, ldk]/[Lk, ldv] with K/V head
//  h / group at kOff / vOff + (h / group)*D. Output [Lq, H*D].
//  bias: optional Tensor of additive score biases for keys biasStart...
// Fused prologue options of this build: qNorm/kNorm (per-head RMSNorm weights, the DiT's
// headNorm), cs (RoPE table with .sinOff) applied to q/k rows < ropeRows, eps.
// textKV (addition to the reference API): { t, off, ld, start } -- key and value rows from
// `start` on come from Tensor t, keys at column off and values at off + H*D of rows with stride
// ld (the DiT's text keys projected for all joint blocks at once); fused path only.
export function attention(gpu, { q, k, v, Lq, Lk, H, D, ldq, ldk, ldv, qOff = 0, kOff = 0, vOff = 0, group = 1,
  causal = false, bias = null, biasStart = 0, out, qNorm = null, kNorm = null, cs = null, ropeRows = 0, eps = 1e-6,
  textKV = null, vPacked = null }) {
  const o = out || gpu.empty([Lq, H * D]);
  // the fused kernel's conditions (app/gpu/ops.js:202-203); otherwise the materialized path's
  // semantics (:211-241), which rejects a key bias
  const aligned = [ldq, ldk, ldv, qOff, kOff, vOff].every((x) => x % 4 === 0);
  if (causal || group !== 1 || D % 32 || D > 128 || !aligned) {
    if (bias) throw new Error("attention: key bias needs the fused kernel");
    if (qNorm || kNorm || cs) throw new Error("attention: fused head norms need the fused kernel");
    if (textKV) throw new Error("attention: a separate text key/value view needs the fused kernel");
    if (vPacked) throw new Error("attention: packed values need the fused kernel");
    if (D > 256) throw new Error(`attention: unsupported head dim ${D}`);
    gpu.run("attn.rows", 4 * Lq * Lk * D * H, () =>
      native.attentionRows(addr(q), addr(k), addr(v), addr(o), Lq, Lk, H, D, ldq, ldk, ldv, H * D, qOff, kOff, vOff,
        group, causal ? 1 : 0));
    return o;
  }
  if (vPacked) {
    // values of keys [0, vPacked.rows) already in vPacked.buf (linear() with opts.vpack)
    const { buf, rows } = vPacked;
    if (buf.vpack.Lk !== Lk || buf.vpack.H !== H || buf.vpack.D !== D) {
      throw new Error("attention: the packed values were made for another shape");
    }
    let kt = null, vt = null, ldText = 0, textStart = 0;
    if (textKV) {
      const base = addr(textKV.t);
      kt = base + BigInt(textKV.off * 4);
      vt = base + BigInt((textKV.off + H * D) * 4);
      ldText = textKV.ld;
      textStart = textKV.start;
    }
    gpu.run("attn.flash", 4 * Lq * Lk * D * H, () =>
      native.attentionVpacked(addr(q), addr(k), addr(v), addr(o), Lq, Lk, H, D, ldq, ldk, ldv, H * D, qOff, kOff,
        vOff, 0, 1 / Math.sqrt(D), addr(bias), biasStart, addr(qNorm), addr(kNorm), eps, cs ? addr(cs) : null,
        cs ? cs.sinOff : 0, cs ? ropeRows : 0, kt, vt, ldText, textStart, addr(buf), rows));
    return o;
  }
  if (textKV) {
    const base = addr(textKV.t);
    const kt = base + BigInt(textKV.off * 4), vt = base + BigInt((textKV.off + H * D) * 4);
    gpu.run("attn.flash", 4 * Lq * Lk * D * H, () =>
      native.attentionText(addr(q), addr(k), addr(v), addr(o), Lq, Lk, H, D, ldq, ldk, ldv, H * D, qOff, kOff, vOff, 0,
        1 / Math.sqrt(D), addr(bias), biasStart, addr(qNorm), addr(kNorm), eps, cs ? addr(cs) : null,
        cs ? cs.sinOff : 0, cs ? ropeRows : 0, kt, vt, textKV.ld, textKV.start));
    return o;
  }
  gpu.run("attn.flash", 4 * Lq * Lk * D * H, () =>
    native.attention(addr(q), addr(k), addr(v), addr(o), 1, Lq, Lk, H, D, ldq, ldk, ldv, H * D, qOff, kOff, vOff, 0,
      0, 0, 0, 0, 1 / Math.sqrt(D), addr(bias), biasStart, 0, addr(qNorm), addr(kNorm), eps,
      cs ? addr(cs) : null, cs ? cs.sinOff : 0, cs ? ropeRows : 0));
  return o;
}

export function conv3x3() {
  throw new Error("conv3x3 (VAE decoder) is not part of this build");
}

export function conv3x3Into() {
  throw new Error("conv3x3 (VAE decoder) is not part of this build");
}

export function groupNorm() {
  throw new Error("groupNorm (VAE decoder) is not part of this build");
}
