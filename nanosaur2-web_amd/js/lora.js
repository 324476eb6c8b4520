// LoRA support for the Node host (app/lora.js): each targeted linear gets a low-rank side path,
// y = W x + sum_i s_i B_i (A_i x), without touching the base weights. Strength changes are
// host-side: the stacked side path of a weight is rebuilt and re-uploaded (a few hundred KB).
//
// File formats and name matching as the reference: PEFT naming ("<module>.lora_A/B.weight" +
// ".alpha") or kohya ("lora_unet_<module_with_underscores>.lora_down/up.weight" + ".alpha"), for
// the DiT and the Gemma3 text encoder; LoKr/LoHa/DoRA are reported as unsupported.
//
// Where the reference (app/gpu/ops.js:70-87) runs two matmuls per LoRA and adds the [M, N] delta
// in the GEMM epilogue, this build stacks every LoRA of a weight into one fp16 pair
//   lora_a [R, K]  (the down-projections; rotated per 256-group for int8 ConvRot weights),
//   lora_b [N, R]  (strength * alpha / r * B_i in its output window, zero elsewhere),
// R = the summed ranks rounded up to 32, and the GEMM kernels start their accumulators at the
// low-rank term (the *_lora entry points of the C ABI).

import { SafeTensors } from "./weights.js";

const norm = (name) => name.replace(/\./g, "_");

const SUFFIXES = [
  [".lora_A.weight", "A"], [".lora_B.weight", "B"],
  [".lora_down.weight", "A"], [".lora_up.weight", "B"],
  [".alpha", "alpha"],
];
const TE_PREFIXES = ["lora_te_", "lora_te1_", "text_encoders.gemma3_270m.transformer.", "text_encoder.", "te."];
const DIT_PREFIXES = ["lora_unet_", "model.diffusion_model.", "diffusion_model.", "base_model.model.", "transformer.", "unet."];
const UNSUPPORTED = /(lokr_|hada_|\.dora_scale|\.diff$|\.diff_b$|\.w_norm|\.b_norm)/;

// Module names of Nanosaur2's linears (DiT and Gemma3), dots as underscores.
const NANOSAUR_MODULE = new RegExp("^(" + [
  "blocks_\\d+_(attn_(qkv_x|kv_y|proj)|mlp_w(12|3))",
  "text_refine_blocks_\\d+_(attn_(qkv|proj)|mlp_w(12|3)|adaLN_modulation_0)",
  "(s|y)_embedder_proj", "t_embedder_mlp_[02]", "shared_encoder_adaLN_0", "y_pool_proj", "sprint_out_proj",
  "final_layer_(linear|adaLN_modulation)",
  "(model_)?layers_\\d+_(self_attn_[qkvo]_proj|mlp_(gate|up|down)_proj)",
].join("|") + ")$");

function suffixOf(key) {
  for (const s of SUFFIXES) if (key.endsWith(s[0])) return s;
  return null;
}

function stripPrefix(name, prefixes) {
  for (const p of prefixes) if (name.startsWith(p)) return [name.slice(p.length), true];
  return [name, false];
}

// A LoRA file's tensor names -> { lora, modules, fits, unsupported } (app/lora.js:32-48).
export function inspectLoraKeys(keys) {
  const modules = new Set();
  let unsupported = 0;
  for (const key of keys) {
    if (UNSUPPORTED.test(key)) { unsupported++; continue; }
    const suf = suffixOf(key);
    if (suf && suf[1] !== "alpha") modules.add(key.slice(0, -suf[0].length));
  }
  let fits = 0;
  for (const m of modules) {
    const [name] = stripPrefix(m, TE_PREFIXES.concat(DIT_PREFIXES));
    if (NANOSAUR_MODULE.test(norm(name))) fits++;
  }
  return { lora: modules.size > 0, modules: modules.size, fits, unsupported };
}

// name (dots as underscores) -> { W, off, n } for every linear reachable from a model object;
// stacked weights register each part (app/lora.js:52-68).
export function linearRegistry(root) {
  const reg = new Map();
  const seen = new Set();
  const walk = (o) => {
    if (!o || typeof o !== "object" || seen.has(o) || ArrayBuffer.isView(o)) return;
    if (o instanceof SafeTensors) return;
    seen.add(o);
    if (o.kind && (o.buf || o.tbuf || o.tglu) && o.N && o.K) {
      if (o.parts) for (const p of o.parts) reg.set(norm(p.name), { W: o, off: p.off, n: p.n });
      else if (o.name) reg.set(norm(o.name), { W: o, off: 0, n: o.N });
      return;
    }
    for (const k of Object.keys(o)) if (k !== "gpu" && k !== "st") walk(o[k]);
  };
  walk(root);
  return reg;
}

// In place: each row's 256-groups times the regular Hadamard H256 (x 1/16), the transform of the
// int8 layers' inputs, so x_r (A H)^T = x A^T (app/lora.js:72-91): four radix-4 stages at strides
// 1, 4, 16, 64 with y = (a + b + c - e, a + b - c + e, a - b + c + e, -a + b + c + e).
export function hadamardRows(data, rows, K) {
  for (let r = 0; r < rows; r++) {
    for (let g = 0; g < K; g += 256) {
      const base = r * K + g;
      for (let stride = 1; stride < 256; stride *= 4) {
        for (let blk = 0; blk < 256; blk += 4 * stride) {
          for (let t = 0; t < stride; t++) {
            const i0 = base + blk + t;
            const a = data[i0], b = data[i0 + stride], c = data[i0 + 2 * stride], e = data[i0 + 3 * stride];
            data[i0] = a + b + c - e;
            data[i0 + stride] = a + b - c + e;
            data[i0 + 2 * stride] = a - b + c + e;
            data[i0 + 3 * stride] = -a + b + c + e;
          }
        }
      }
      for (let i = 0; i < 256; i++) data[base + i] *= 0.0625;
    }
  }
}

function findTarget(module, regs) {
  let [name, te] = stripPrefix(module, TE_PREFIXES);
  if (!te) name = stripPrefix(name, DIT_PREFIXES)[0];
  const key = norm(name);
  const order = te ? [regs.te] : [regs.dit, regs.te];
  for (const reg of order) {
    if (!reg) continue;
    if (reg.has(key)) return reg.get(key);
    if (reg.has("model_" + key)) return reg.get("model_" + key); // kohya TE names omit "model."
  }
  return null;
}

// Parses a LoRA file (a path or an open SafeTensors) for the given registries ({ dit, te }).
// Returns { modules: [{ target, A, B, r, alphaScale }], matched, total, unsupported, skipped }
// with A (rotated for int8 targets) and B as host Float32Arrays (app/lora.js:96-131).
export async function loadLora(source, regs) {
  const st = typeof source === "string" ? await SafeTensors.open(source) : source;
  const groups = new Map();
  let unsupported = 0;
  for (const key of Object.keys(st.header)) {
    if (UNSUPPORTED.test(key)) { unsupported++; continue; }
    const suf = suffixOf(key);
    if (!suf) continue;
    const module = key.slice(0, -suf[0].length);
    if (!groups.has(module)) groups.set(module, {});
    groups.get(module)[suf[1]] = key;
  }
  const modules = [];
  let skipped = 0;
  for (const [module, keys] of groups) {
    if (!keys.A || !keys.B) { skipped++; continue; }
    const target = findTarget(module, regs);
    const aInfo = st.info(keys.A), bInfo = st.info(keys.B);
    const r = aInfo.shape[0];
    if (!target || aInfo.shape[1] !== target.W.K || bInfo.shape[0] !== target.n || bInfo.shape[1] !== r) { skipped++; continue; }
    const A = Float32Array.from(await st.f32(keys.A)); // own copy: rotated in place for int8 layers
    if (target.W.kind === "i8") hadamardRows(A, r, target.W.K);
    const B = Float32Array.from(await st.f32(keys.B));
    const alpha = keys.alpha ? (await st.f32(keys.alpha))[0] : null;
    modules.push({ target, A, B, r, alphaScale: alpha ? alpha / r : 1 });
  }
  if (typeof source === "string") st.close();
  return { modules, matched: modules.length, total: groups.size, unsupported, skipped };
}

// Releases the stacked side paths built for a registry's weights.
function dropPacks(regs) {
  for (const reg of [regs.dit, regs.te]) {
    if (!reg) continue;
    for (const { W } of reg.values()) {
      if (W.loraPack) {
        W.loraPack.a.destroy();
        W.loraPack.b.destroy();
        W.loraPack = null;
      }
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

// Host arrays of a weight's stacked side path: { a: fp32 [R, K], b: fp32 [N, R], R }.
export function stackLora(W) {
  const rs = W.lora.reduce((s, e) => s + e.r, 0);
  const R = Math.ceil(rs / 32) * 32;
  if (R > 256) throw new Error(`${W.name}: stacked LoRA rank ${rs} exceeds 256`);
  const a = new Float32Array(R * W.K);
  const b = new Float32Array(W.N * R);
  let r0 = 0;
  for (const e of W.lora) {
    a.set(e.A, r0 * W.K);
    for (let i = 0; i < e.n; i++) {
      const row = (e.off + i) * R + r0;
      for (let k = 0; k < e.r; k++) b[row + k] = e.scale * e.B[i * e.r + k];
    }
    r0 += e.r;
  }
  return { a, b, R };
}

// The device side path of W for the *_lora entry points ([loraA, loraB, loraR]), built on first
// use after attachLoras; [null, null, 0] without LoRA.
export function loraArgs(gpu, W) {
  if (!W.lora || !W.lora.length) return [null, null, 0];
  if (!W.loraPack) {
    const { a, b, R } = stackLora(W);
    W.loraPack = { a: gpu.upload(f32ToF16Bits(a)), b: gpu.upload(f32ToF16Bits(b)), R };
  }
  return [W.loraPack.a.ptr, W.loraPack.b.ptr, W.loraPack.R];
}
