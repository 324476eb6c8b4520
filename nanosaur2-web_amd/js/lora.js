// LoRA side paths for the Node host: every linear a LoRA file names gets
// y = W x + sum_i s_i B_i (A_i x), and the base weights stay as they are (the behaviour of
// app/lora.js). Files use PEFT names ("<module>.lora_A/B.weight" + ".alpha") or kohya names
// ("lora_unet_<module_with_underscores>.lora_down/up.weight" + ".alpha"), for the DiT and the
// Gemma3 text encoder; LoKr / LoHa / DoRA tensors are counted as unsupported.
//
// How it is organised here:
//  * each model lists its linears (linears()), and linearRegistry maps the canonical module key
//    (dots as underscores) to a weight slice { W, off, n } -- a stacked weight such as Gemma3's
//    q|k|v has one slice per part;
//  * loadLora reads a file into host arrays and resolves each module to a slice; attachLoras
//    hands them to their weights with a strength;
//  * the first launch of a weight after that builds its side paths on the device
//    (loraLaunches): the LoRAs of a row window of the weight stacked into one fp16 pair,
//    lora_a [R, K] and lora_b [n, R] (strength * alpha / r * B_i in its output rows, zero
//    elsewhere), R the summed ranks rounded up to 32 and at most MAX_RANK. A weight is one
//    window; a stacked weight (Gemma3's q|k|v, the DiT's kv_y of all joint blocks) is cut into
//    windows of whole parts when its parts' ranks do not fit one side path, and linear() then
//    launches once per window. The GEMM kernels start their accumulators at the low-rank term
//    (the *_lora entry points of the C ABI) where the reference runs two more matmuls per LoRA
//    and adds an [M, N] delta (app/gpu/ops.js:70-87).
//  * int8 ConvRot weights take rotated inputs x H, and x A^T = (x H)(A H)^T, so their lora_a
//    rows are rotated on the device by the kernel that rotates the activations
//    (app/lora.js:72-91 rotates them on the host).

import { SafeTensors } from "./weights.js";
import { addr, DeviceBuffer } from "./device.js";
import { native } from "./native.js";

// ---- names (format data: the tensor roles, trainer prefixes and unsupported markers) ---------

// "<module>.<role>": role A (down-projection), B (up-projection) or the alpha scalar
const ROLE = /^(.+)\.(?:(lora_A|lora_down)\.weight|(lora_B|lora_up)\.weight|(alpha))$/;
const TE_PREFIXES = ["lora_te_", "lora_te1_", "text_encoders.gemma3_270m.transformer.", "text_encoder.", "te."];
const DIT_PREFIXES = ["lora_unet_", "model.diffusion_model.", "diffusion_model.", "base_model.model.", "transformer.", "unet."];
const UNSUPPORTED = /(lokr_|hada_|\.dora_scale|\.diff$|\.diff_b$|\.w_norm|\.b_norm)/;

// Module keys of Nanosaur2's linears (DiT and Gemma3).
const NANOSAUR_MODULE = new RegExp("^(" + [
  "blocks_\\d+_(attn_(qkv_x|kv_y|proj)|mlp_w(12|3))",
  "text_refine_blocks_\\d+_(attn_(qkv|proj)|mlp_w(12|3)|adaLN_modulation_0)",
  "(s|y)_embedder_proj", "t_embedder_mlp_[02]", "shared_encoder_adaLN_0", "y_pool_proj", "sprint_out_proj",
  "final_layer_(linear|adaLN_modulation)",
  "(model_)?layers_\\d+_(self_attn_[qkvo]_proj|mlp_(gate|up|down)_proj)",
].join("|") + ")$");

const keyOf = (dotted) => dotted.split(".").join("_");

// { module, role } of a LoRA tensor name, or null for a tensor that is not part of a LoRA pair.
function parseName(name) {
  const m = ROLE.exec(name);
  if (!m) return null;
  return { module: m[1], role: m[2] ? "A" : m[3] ? "B" : "alpha" };
}

// A module name without its trainer prefix: { key, textEncoder } -- a text-encoder prefix
// confines the lookup to the text encoder.
function canonical(module) {
  const te = TE_PREFIXES.find((p) => module.startsWith(p));
  const other = te ? "" : DIT_PREFIXES.find((p) => module.startsWith(p)) || "";
  return { key: keyOf(module.slice((te || other).length)), textEncoder: !!te };
}

// The tensors of a LoRA file grouped by module: { groups: Map(module -> {A, B, alpha}), unsupported }.
function groupTensors(names) {
  const groups = new Map();
  let unsupported = 0;
  for (const name of names) {
    if (UNSUPPORTED.test(name)) {
      unsupported++;
      continue;
    }
    const p = parseName(name);
    if (!p) continue;
    const g = groups.get(p.module) || {};
    g[p.role] = name;
    groups.set(p.module, g);
  }
  return { groups, unsupported };
}

// A LoRA file's tensor names -> { lora, modules, fits, unsupported }: is it a LoRA this build
// applies, and how many of its modules have Nanosaur2's names (app/lora.js:32-48).
export function inspectLoraKeys(names) {
  const { groups, unsupported } = groupTensors(names);
  const modules = [...groups].filter(([, g]) => g.A || g.B).map(([m]) => m);
  const fits = modules.filter((m) => NANOSAUR_MODULE.test(canonical(m).key)).length;
  return { lora: modules.length > 0, modules: modules.length, fits, unsupported };
}

// ---- registry ------------------------------------------------------------------------------

// The named slices of a weight: one per part of a stacked weight, else the whole weight.
export function weightSlices(W) {
  if (W.parts) return W.parts.map((p) => ({ name: p.name, W, off: p.off, n: p.n }));
  return [{ name: W.name, W, off: 0, n: W.N }];
}

// module key -> { W, off, n } over the linears a model lists (model.linears()).
export function linearRegistry(model) {
  const reg = new Map();
  for (const W of model.linears()) for (const s of weightSlices(W)) reg.set(keyOf(s.name), s);
  return reg;
}

// The weight slice a LoRA module targets in regs ({ dit, te }), or null. A module without a
// text-encoder prefix is looked up in the DiT first; kohya text-encoder names leave out the
// model's "model." root, so "model_" + key is tried as well.
function resolve(module, regs) {
  const { key, textEncoder } = canonical(module);
  const where = textEncoder ? [regs.te] : [regs.dit, regs.te];
  for (const reg of where) {
    if (!reg) continue;
    const hit = reg.get(key) || reg.get("model_" + key);
    if (hit) return hit;
  }
  return null;
}

// ---- loading -------------------------------------------------------------------------------

// Parses a LoRA file (a path or an open SafeTensors) for the registries { dit, te }. Returns
// { modules: [{ target, A, B, r, alphaScale }], matched, total, unsupported, skipped }, A [r, K]
// and B [n, r] as host Float32Arrays (app/lora.js:96-131). A module is skipped when it lacks
// A or B, names no linear of the model, or its shapes do not fit the slice it names.
export async function loadLora(source, regs) {
  const st = typeof source === "string" ? await SafeTensors.open(source) : source;
  try {
    const { groups, unsupported } = groupTensors(st.names());
    const modules = [];
    for (const [module, g] of groups) {
      const target = g.A && g.B ? resolve(module, regs) : null;
      if (!target) continue;
      const [r, k] = st.info(g.A).shape;
      const [n, rb] = st.info(g.B).shape;
      if (k !== target.W.K || n !== target.n || rb !== r) continue;
      const A = Float32Array.from(await st.f32(g.A));
      const B = Float32Array.from(await st.f32(g.B));
      const alpha = g.alpha ? (await st.f32(g.alpha))[0] : null;
      modules.push({ target, A, B, r, alphaScale: alpha ? alpha / r : 1 });
    }
    return { modules, matched: modules.length, total: groups.size, unsupported, skipped: groups.size - modules.length };
  } finally {
    if (typeof source === "string") st.close();
  }
}

// Releases the device side paths built for a registry's weights.
function dropPacks(regs) {
  for (const reg of [regs.dit, regs.te]) {
    if (!reg) continue;
    for (const { W } of reg.values()) {
      if (!W.loraPacks) continue;
      for (const p of W.loraPacks) {
        if (!p.args) continue;
        p.a.destroy();
        p.b.destroy();
      }
      W.loraPacks = null;
    }
  }
}

// Nothing of a parsed LoRA lives on the device (its packs belong to the weights).
export function destroyLora() {}

// Replace every LoRA side path in the registries with the given [{ lora, strength }]
// (app/lora.js:144-152).
export function attachLoras(regs, active) {
  dropPacks(regs);
  for (const reg of [regs.dit, regs.te]) if (reg) for (const { W } of reg.values()) W.lora = [];
  for (const { lora, strength } of active) {
    if (!strength) continue;
    for (const m of lora.modules) {
      m.target.W.lora.push({ A: m.A, B: m.B, r: m.r, scale: strength * m.alphaScale, off: m.target.off, n: m.target.n });
    }
  }
}

// ---- the stacked side path -----------------------------------------------------------------

// fp32 -> fp16 bit patterns, round to nearest even (subnormals kept, overflow to infinity).
export function f32ToF16Bits(f) {
  const out = new Uint16Array(f.length);
  const fb = new Float32Array(1);
  const ub = new Uint32Array(fb.buffer);
  for (let i = 0; i < f.length; i++) {
    fb[0] = f[i];
    const x = ub[0];
    const sign = (x >>> 16) & 0x8000;
    const e = (x >>> 23) & 0xff;
    let m = x & 0x7fffff;
    if (e === 0xff) { out[i] = sign | 0x7c00 | (m ? 0x200 : 0); continue; }
    let he = e - 127 + 15;
    if (he >= 0x1f) { out[i] = sign | 0x7c00; continue; }
    if (he <= 0) {
      if (he < -10) { out[i] = sign; continue; }
      m |= 0x800000;
      const shift = 14 - he;
      let hm = m >>> shift;
      const rem = m & ((1 << shift) - 1), half = 1 << (shift - 1);
      if (rem > half || (rem === half && (hm & 1))) hm++;
      out[i] = sign | hm;
      continue;
    }
    let hm = m >>> 13;
    const rem = m & 0x1fff;
    if (rem > 0x1000 || (rem === 0x1000 && (hm & 1))) {
      hm++;
      if (hm === 0x400) { hm = 0; he++; if (he >= 0x1f) { out[i] = sign | 0x7c00; continue; } }
    }
    out[i] = sign | (he << 10) | hm;
  }
  return out;
}

// Largest stacked rank of one side path (the GEMM epilogues' low-rank term).
export const MAX_RANK = 256;

const roundRank = (r) => Math.ceil(r / 32) * 32;
const weightLabel = (W) => W.name || (W.parts ? W.parts.map((p) => p.name).join("+") : "linear");

// The row windows of W that share one side path: [{ off, n, entries }]. A weight without parts
// is one window. The parts of a stacked weight stay together while their ranks fit MAX_RANK;
// past that a new window starts at the next part, so each window is a run of whole parts
// (the reference applies each LoRA on its own, with no rank limit: app/gpu/ops.js:70-87).
export function loraWindows(W) {
  const lora = W.lora || [];
  const parts = W.parts || [{ name: W.name, off: 0, n: W.N }];
  const wins = [];
  let cur = null;
  for (const p of parts) {
    const entries = lora.filter((e) => e.off >= p.off && e.off < p.off + p.n);
    const r = entries.reduce((s, e) => s + e.r, 0);
    if (roundRank(r) > MAX_RANK) {
      throw new Error(`${p.name || weightLabel(W)}: LoRA rank ${r} on one linear exceeds ${MAX_RANK}`);
    }
    if (cur && roundRank(cur.rank + r) <= MAX_RANK) {
      cur.n += p.n;
      cur.rank += r;
      cur.entries.push(...entries);
    } else {
      cur = { off: p.off, n: p.n, rank: r, entries };
      wins.push(cur);
    }
  }
  return wins.map(({ off, n, entries }) => ({ off, n, entries }));
}

// Host arrays of one side path: { a: fp32 [R, K] (not rotated), b: fp32 [n, R], R } over the
// row window win of W (the whole weight by default).
export function stackLora(W, win = { off: 0, n: W.N, entries: W.lora }) {
  const rs = win.entries.reduce((s, e) => s + e.r, 0);
  const R = roundRank(rs);
  if (R > MAX_RANK) throw new Error(`${weightLabel(W)}: stacked LoRA rank ${rs} exceeds ${MAX_RANK}`);
  const a = new Float32Array(R * W.K);
  const b = new Float32Array(win.n * R);
  let r0 = 0;
  for (const e of win.entries) {
    a.set(e.A, r0 * W.K);
    for (let i = 0; i < e.n; i++) {
      const row = (e.off - win.off + i) * R + r0;
      for (let k = 0; k < e.r; k++) b[row + k] = e.scale * e.B[i * e.r + k];
    }
    r0 += e.r;
  }
  return { a, b, R };
}

// The device side path of one window of W: lora_b uploaded as fp16; lora_a as fp16 too, for an
// int8 weight rotated per 256-group on the way by the activation rotation kernel (fp32 rows in a
// pooled staging tensor, rotated and rounded to fp16 into the persistent buffer).
function buildPack(gpu, W, win) {
  const { a, b, R } = stackLora(W, win);
  let aBuf;
  if (W.kind === "i8") {
    const bytes = R * W.K * 2;
    aBuf = new DeviceBuffer(native.malloc(bytes), bytes, false);
    const staged = gpu.fromArray(a, [R, W.K]);
    native.rotateF16(addr(staged), W.K, aBuf.ptr, W.K, R, W.K, 0);
    staged.release();
  } else {
    aBuf = gpu.upload(f32ToF16Bits(a));
  }
  return { a: aBuf, b: gpu.upload(f32ToF16Bits(b)), R };
}

// The launches a linear over W makes: [{ off, n, args }], args = [loraA, loraB, loraR] for the
// *_lora entry points over output rows [off, off + n) of W. One launch over the whole weight
// without LoRA ([null, null, 0]) or when its LoRAs fit one side path; the side paths are built
// on first use after attachLoras.
export function loraLaunches(gpu, W) {
  if (!W.lora || !W.lora.length) return [{ off: 0, n: W.N, args: [null, null, 0] }];
  if (!W.loraPacks) {
    W.loraPacks = loraWindows(W).map((win) => {
      if (!win.entries.length) return { off: win.off, n: win.n, args: [null, null, 0] };
      const p = buildPack(gpu, W, win);
      return { off: win.off, n: win.n, a: p.a, b: p.b, args: [p.a.ptr, p.b.ptr, p.R] };
    });
  }
  return W.loraPacks;
}

// [loraA, loraB, loraR] of W for a launch that covers the whole weight (the fused GLU and
// packed-value launches); [null, null, 0] without LoRA.
export function loraArgs(gpu, W) {
  const ls = loraLaunches(gpu, W);
  if (ls.length !== 1) throw new Error(`${weightLabel(W)}: its LoRAs need ${ls.length} side paths; this launch takes one`);
  return ls[0].args;
}
