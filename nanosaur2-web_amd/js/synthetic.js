// Seeded random-init weights of the Nanosaur2 DiT architecture, produced in memory with the
// weight-source interface of weights.js (has / vector / linear). Block linears are int8
// ConvRot (U{-127..127} with per-row scales U[1e-3, 1e-2]); the other linears, norms and
// adaLN offsets are bf16 / fp32 ~ N(0, 0.02). Used for timing runs, where values do not
// matter; parity runs load the same architecture from a safetensors file instead.

const D = 1536;

// name -> { shape, kind: "i8" | "bf16" | "vec" } for the real model (MLP width I = 4096).
export function ditSpec({ I = 4096, blocks = 18, textBlocks = 2, ctx = 640 } = {}) {
  const s = new Map();
  const bf = (n, shape) => s.set(n, { shape, kind: "bf16" });
  const i8 = (n, shape) => s.set(n, { shape, kind: "i8" });
  const vec = (n, len) => s.set(n, { shape: [len], kind: "vec" });
  bf("s_embedder.proj.weight", [D, 64]);
  bf("t_embedder.mlp.0.weight", [D, 256]);
  bf("t_embedder.mlp.2.weight", [D, D]);
  bf("y_embedder.proj.weight", [D, ctx]);
  vec("y_embedder.norm.weight", D);
  bf("y_pool_proj.weight", [D, D]);
  bf("shared_encoder_adaLN.0.weight", [6 * D, D]);
  bf("sprint_out_proj.weight", [D, D]);
  for (let i = 0; i < textBlocks; i++) {
    const p = `text_refine_blocks.${i}.`;
    bf(p + "adaLN_modulation.0.weight", [6 * D, D]);
    vec(p + "norm1.weight", D);
    vec(p + "norm2.weight", D);
    i8(p + "attn.qkv.weight", [3 * D, D]);
    vec(p + "attn.q_norm.weight", 96);
    vec(p + "attn.k_norm.weight", 96);
    i8(p + "attn.proj.weight", [D, D]);
    i8(p + "mlp.w12.weight", [2 * I, D]);
    i8(p + "mlp.w3.weight", [D, I]);
  }
  for (let i = 0; i < blocks; i++) {
    const p = `blocks.${i}.`;
    vec(`encoder_adaLN_offsets.${i}`, 6 * D);
    vec(p + "norm1.weight", D);
    vec(p + "norm2.weight", D);
    i8(p + "attn.qkv_x.weight", [3 * D, D]);
    if (i % 2 === 0) i8(p + "attn.kv_y.weight", [2 * D, D]);
    vec(p + "attn.q_norm.weight", 96);
    vec(p + "attn.k_norm.weight", 96);
    i8(p + "attn.proj.weight", [D, D]);
    i8(p + "mlp.w12.weight", [2 * I, D]);
    i8(p + "mlp.w3.weight", [D, I]);
  }
  bf("final_layer.adaLN_modulation.weight", [2 * D, D]);
  bf("final_layer.linear.weight", [64, D]);
  return s;
}

// name -> spec for the Gemma3-270M text encoder (app/models/gemma3.js:13-45): bf16 linears and
// norms, the [262144, 640] embedding table (its rows are generated on demand).
export function gemmaSpec({ layers = 17, vocab = 262144 } = {}) {
  const s = new Map();
  const bf = (n, shape) => s.set(n, { shape, kind: "bf16" });
  const vec = (n, len) => s.set(n, { shape: [len], kind: "vec" });
  s.set("model.embed_tokens.weight", { shape: [vocab, 640], kind: "table" });
  for (let i = 0; i < layers; i++) {
    const p = `model.layers.${i}.`;
    for (const n of ["input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm", "post_feedforward_layernorm"]) vec(p + n + ".weight", 640);
    vec(p + "self_attn.q_norm.weight", 256);
    vec(p + "self_attn.k_norm.weight", 256);
    bf(p + "self_attn.q_proj.weight", [1024, 640]);
    bf(p + "self_attn.k_proj.weight", [256, 640]);
    bf(p + "self_attn.v_proj.weight", [256, 640]);
    bf(p + "self_attn.o_proj.weight", [640, 1024]);
    bf(p + "mlp.gate_proj.weight", [2048, 640]);
    bf(p + "mlp.up_proj.weight", [2048, 640]);
    bf(p + "mlp.down_proj.weight", [640, 2048]);
  }
  vec("model.norm.weight", 640);
  return s;
}

// xorshift128+-style generator on 32-bit halves (seeded per tensor name)
function rng(seed, name) {
  let h = (seed ^ 0x9e3779b9) >>> 0;
  for (let i = 0; i < name.length; i++) h = Math.imul(h ^ name.charCodeAt(i), 0x01000193) >>> 0;
  let a = h || 1;
  let b = (Math.imul(h, 0x85ebca6b) ^ 0x27d4eb2f) >>> 0 || 2;
  return () => {
    let t = a;
    const s = b;
    a = s;
    t ^= t << 11;
    t ^= t >>> 8;
    b = (t ^ s ^ (s >>> 19)) >>> 0;
    return b;
  };
}

export class SyntheticWeights {
  constructor(seed = 3, opts = {}) {
    this.seed = seed;
    this.spec = opts.gemma ? gemmaSpec(opts) : ditSpec(opts);
  }
  has(name) {
    if (name.endsWith("weight_scale")) return this.spec.has(name.replace(/_scale$/, ""));
    return this.spec.has(name);
  }
  normal(name, n, std) {
    const r = rng(this.seed, name);
    const out = new Float32Array(n);
    for (let i = 0; i < n; i++) {
      // Irwin-Hall(4) approximation of a normal: var = 4/12
      const u = ((r() >>> 8) + (r() >>> 8) + (r() >>> 8) + (r() >>> 8)) / 16777216 - 2;
      out[i] = u * Math.sqrt(3) * std;
    }
    return out;
  }
  async vector(gpu, name, add = 0) {
    const e = this.spec.get(name);
    if (!e) throw new Error(`missing tensor ${name}`);
    const v = this.normal(name, e.shape[0], 0.02);
    return gpu.upload(add ? v.map((x) => x + add) : v);
  }
  // rows of a table (embeddings), each generated from its own seed
  async rows(name, ids) {
    const e = this.spec.get(name);
    if (!e) throw new Error(`missing tensor ${name}`);
    const dim = e.shape[1];
    const out = new Float32Array(ids.length * dim);
    ids.forEach((id, i) => out.set(this.normal(`${name}#${id}`, dim, 1.0), i * dim));
    return out;
  }
  async linear(gpu, base) {
    const e = this.spec.get(base + "weight");
    if (!e) throw new Error(`missing tensor ${base}weight`);
    const [N, K] = e.shape;
    const name = base.replace(/\.$/, "");
    if (e.kind === "i8") {
      const r = rng(this.seed, base);
      const q = new Int8Array(N * K);
      for (let i = 0; i < q.length; i += 4) {
        const v = r();
        for (let j = 0; j < 4 && i + j < q.length; j++) q[i + j] = ((v >>> (8 * j)) & 0xff) % 255 - 127;
      }
      const rs = rng(this.seed, base + "scale");
      const scale = new Float32Array(N);
      for (let i = 0; i < N; i++) scale[i] = 1e-3 + 9e-3 * (rs() / 4294967296);
      return { kind: "i8", N, K, buf: gpu.upload(q), scale: gpu.upload(scale), bias: null, name };
    }
    const f = this.normal(base, N * K, 0.02);
    const bits = new Uint32Array(f.buffer);
    const bf = new Uint16Array(N * K);
    for (let i = 0; i < bf.length; i++) bf[i] = bits[i] >>> 16;
    return { kind: "bf16", N, K, buf: gpu.upload(bf), bias: null, name };
  }
}
