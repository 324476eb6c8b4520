// Gemma3-270M text encoder as Nanosaur2 uses it (app/models/gemma3.js): the hidden state after
// the 17th of 18 layers with the final norm applied (ComfyUI layer="hidden", layer_idx=-2).
//
// Embeddings scaled by sqrt(640); RMSNorm weights stored as w - 1 (+1 at load); norms before and
// after both attention and MLP; q/k norms with split-half RoPE; one K/V head for the four query
// heads (causal, through ops.attention's materialized-path kernel); GELU(tanh)-gated MLP. Every
// 6th layer is global (RoPE theta 1e6), the others local (theta 1e4; their 512-token window
// never applies at <= 256 tokens).

import * as ops from "./ops.js";
import { concatLinears } from "./weights.js";
import { ropeTable } from "./common.js";

export const GEMMA = { layers: 18, hidden: 640, heads: 4, kvHeads: 1, headDim: 256, globalEvery: 6 };
const RUN = GEMMA.layers - 1; // layers needed for the penultimate hidden state

// One decoder layer's tensors under the checkpoint's names (app/models/gemma3.js:17-41 reads
// the same set): its norm vectors, and its linears with q|k|v and gate|up stacked into one
// weight each (concatLinears), so each pair of projections is one GEMM.
const LAYER_NORMS = {
  inNorm: "input_layernorm",
  postAttnNorm: "post_attention_layernorm",
  preMlpNorm: "pre_feedforward_layernorm",
  postMlpNorm: "post_feedforward_layernorm",
  qn: "self_attn.q_norm",
  kn: "self_attn.k_norm",
};
const LAYER_LINEARS = {
  qkv: ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"],
  o: ["self_attn.o_proj"],
  gateUp: ["mlp.gate_proj", "mlp.up_proj"],
  down: ["mlp.down_proj"],
};

async function loadLayer(gpu, st, i) {
  const prefix = `model.layers.${i}.`;
  // every GEMMA.globalEvery-th layer attends globally, the others through the sliding window
  const layer = { global: (i + 1) % GEMMA.globalEvery === 0 };
  for (const [key, name] of Object.entries(LAYER_NORMS)) layer[key] = await st.vector(gpu, `${prefix}${name}.weight`, 1);
  for (const [key, parts] of Object.entries(LAYER_LINEARS)) {
    const ws = [];
    for (const part of parts) ws.push(await st.linear(gpu, `${prefix}${part}.`));
    layer[key] = ws.length > 1 ? concatLinears(gpu, ws) : ws[0];
  }
  return layer;
}

export class Gemma3 {
  // st: { linear, vector, rows, has } (weights.js SafeTensors or the synthetic source)
  static async load(gpu, st, onProgress) {
    const m = new Gemma3(gpu, st);
    m.layers = [];
    for (let i = 0; i < RUN; i++) {
      const l = await loadLayer(gpu, st, i);
      // every linear re-tiled as fp16 (next to its row-major copy): q/k/v and gate/up take the
      // tiled operands the row kernels write, o_proj and down the fused projections of the
      // attention and of the GLU
      for (const W of [l.qkv, l.o, l.gateUp, l.down]) if (ops.tileablePlain(W)) ops.tileWeight(gpu, W);
      m.layers.push(l);
      if (onProgress) onProgress((i + 1) / RUN);
    }
    m.norm = await st.vector(gpu, "model.norm.weight", 1);
    return m;
  }

  constructor(gpu, st) {
    this.gpu = gpu;
    this.st = st; // embedding rows are gathered from the source on demand
  }

  // Every linear weight of the stack (LoRA targets; q|k|v and gate|up are stacked weights
  // whose parts keep their module names).
  linears() {
    return this.layers.flatMap((l) => [l.qkv, l.o, l.gateUp, l.down]);
  }

  // Token ids -> Tensor [L, 640] on the device.
  async encode(ids) {
    const x = this.embed(await this.st.rows("model.embed_tokens.weight", ids), ids.length);
    return this.encodeEmbedded(x);
  }

  // Host embedding rows [L, 640] -> scaled device tensor.
  embed(rows, L) {
    const scale = Math.sqrt(GEMMA.hidden);
    const e = new Float32Array(rows.length);
    for (let i = 0; i < rows.length; i++) e[i] = rows[i] * scale;
    return this.gpu.fromArray(e, [L, GEMMA.hidden]);
  }

  // The layer stack on a device tensor x [L, 640] (released here); returns the normed output.
  // Each sublayer's output projection, post-norm, residual add and the norm after it run as one
  // linearAddRmsnorm (a GEMM and a row kernel).
  encodeEmbedded(x) {
    const gpu = this.gpu;
    const { hidden: D, heads: H, kvHeads: KH, headDim: HD } = GEMMA;
    const Lt = x.shape[0];
    const qkvW = (H + 2 * KH) * HD;
    const [csLocal, csGlobal] = this.ropeTables(Lt);
    const noLora = (W) => !(W.lora && W.lora.length);
    // a linear whose input the previous row kernel can write as the tiled fp16 operand takes
    // the tiled path (a LoRA on it keeps the row-major path and its fp32 input)
    const tiled = ops.tiledPathOk;
    const mlpFused = (l) => Number.isInteger(l.gateUp.N / (2 * ops.GLU_DOWN_GROUP)) && l.down.tbuf && noLora(l.down) &&
      l.gateUp.kind === "bf16" && noLora(l.gateUp);
    // the layer input: fp32 h, or hT as the tiled operand of its q/k/v projection
    let h = ops.rmsnorm(gpu, x, this.layers[0].inNorm, D);
    let hT = null;
    if (tiled(this.layers[0].qkv)) {
      hT = ops.toTiled(gpu, h);
      h.release();
      h = null;
    }
    this.layers.forEach((l, i) => {
      const cs = l.global ? csGlobal : csLocal;
      // [Lt, q 1024 | k 256 | v 256], the q heads and then the k head normed and rotated in the
      // projection's split-K sum (on the fused paths the k and v heads are stored as fp16, the
      // attention's operand type)
      let qkv;
      if (hT) {
        qkv = ops.linearHeadNormTiled(gpu, hT, l.qkv, l.qn, H, l.kn, KH, { D: HD, cs });
        hT.release();
        hT = null;
      } else {
        qkv = ops.linearHeadNorm(gpu, h, l.qkv, l.qn, H, l.kn, KH, { D: HD, cs, f16kv: true });
        h.release();
        h = null;
      }
      const mlpTiled = mlpFused(l) && tiled(l.gateUp);
      let h2 = null;
      let h2T = null;
      if (qkv.f16kv && l.o.tbuf && noLora(l.o)) {
        // the attention and o_proj in one launch (each head's share of the projection), the
        // shares summed by the post-norm's row kernel
        const part = ops.attentionRowsF16kvOproj(gpu, {
          q: qkv, kv: qkv, Lq: Lt, Lk: Lt, H, D: HD, ldq: qkvW, qOff: 0, kOff: qkv.f16kv.off,
          vOff: qkv.f16kv.off + KH * HD, ldkv: qkv.f16kv.ld, group: H / KH, causal: true, W: l.o,
        });
        qkv.release();
        if (mlpTiled) h2T = ops.partsAddRmsnormTiled(gpu, part, H, l.o.bias, x, l.postAttnNorm, l.preMlpNorm);
        else h2 = ops.partsAddRmsnorm(gpu, part, H, l.o.bias, x, l.postAttnNorm, l.preMlpNorm);
        part.release();
      } else {
        const a = qkv.f16kv
          ? ops.attentionRowsF16kv(gpu, {
            q: qkv, kv: qkv, Lq: Lt, Lk: Lt, H, D: HD, ldq: qkvW, qOff: 0, kOff: qkv.f16kv.off,
            vOff: qkv.f16kv.off + KH * HD, ldkv: qkv.f16kv.ld, group: H / KH, causal: true,
          })
          : ops.attention(gpu, {
            q: qkv, k: qkv, v: qkv, Lq: Lt, Lk: Lt, H, D: HD, ldq: qkvW, ldk: qkvW, ldv: qkvW,
            qOff: 0, kOff: H * HD, vOff: (H + KH) * HD, group: H / KH, causal: true,
          });
        qkv.release();
        h2 = ops.linearAddRmsnorm(gpu, a, l.o, x, l.postAttnNorm, l.preMlpNorm);
        a.release();
        if (mlpTiled) {
          h2T = ops.toTiled(gpu, h2);
          h2.release();
          h2 = null;
        }
      }
      const last = i + 1 === this.layers.length;
      const next = last ? this.norm : this.layers[i + 1].inNorm;
      // the next layer's q/k/v input as its tiled operand, or fp32 (and the final norm's output)
      const nextTiled = !last && tiled(this.layers[i + 1].qkv);
      if (mlpFused(l)) {
        // the GLU's row kernel writes the down projection's shares per column group, summed by
        // the post-norm's row kernel
        const shares = l.gateUp.N / (2 * ops.GLU_DOWN_GROUP);
        const part = h2T ? ops.linearGluDownTiled(gpu, h2T, l.gateUp, l.down, "gelu_tanh")
          : ops.linearGluDown(gpu, h2, l.gateUp, l.down, "gelu_tanh");
        if (h2T) h2T.release();
        if (h2) h2.release();
        if (nextTiled) hT = ops.partsAddRmsnormTiled(gpu, part, shares, l.down.bias, x, l.postMlpNorm, next);
        else h = ops.partsAddRmsnorm(gpu, part, shares, l.down.bias, x, l.postMlpNorm, next);
        part.release();
      } else {
        const g = ops.linearGlu(gpu, h2, l.gateUp, "gelu_tanh");
        h2.release();
        h = ops.linearAddRmsnorm(gpu, g, l.down, x, l.postMlpNorm, next);
        g.release();
        if (nextTiled) {
          hT = ops.toTiled(gpu, h);
          h.release();
          h = null;
        }
      }
    });
    x.release();
    return h; // the final norm of the last layer's output
  }

  // The local (theta 1e4) and global (1e6) RoPE tables for L tokens, built once per L (they
  // depend on L only; keeping them also keeps host uploads out of a captured encode).
  ropeTables(L) {
    if (!this.rope) this.rope = new Map();
    if (!this.rope.has(L)) {
      const { headDim: HD } = GEMMA;
      this.rope.set(L, [ropeTable(this.gpu, L, HD, 1e4), ropeTable(this.gpu, L, HD, 1e6)]);
    }
    return this.rope.get(L);
  }

  // One encode of L tokens recorded as a HIP graph. Returns { input [L, 640], output [L, 640],
  // launch(), destroy() }: write the scaled embeddings into input, launch, then read output.
  // The graph copies input before the stack (which updates its input in place), so input
  // survives a replay.
  captureEncode(L) {
    const gpu = this.gpu;
    const input = gpu.empty([L, GEMMA.hidden]);
    gpu.write(input.buf, new Float32Array(L * GEMMA.hidden));
    const g = gpu.capture(() => this.encodeEmbedded(ops.elementwise(gpu, "copy", input)));
    return {
      input,
      output: g.result,
      launch: g.launch,
      destroy: () => {
        g.destroy();
        g.result.release();
        input.release();
      },
    };
  }

  unload() {
    if (this.rope) for (const ts of this.rope.values()) for (const t of ts) t.release();
    this.rope = null;
    const seen = new Set();
    const walk = (o) => {
      if (!o || typeof o !== "object" || seen.has(o)) return;
      seen.add(o);
      if (typeof o.destroy === "function" && o.ptr !== undefined) { o.destroy(); return; }
      for (const k of Object.keys(o)) if (k !== "gpu" && k !== "st") walk(o[k]);
    };
    walk(this.layers);
    walk(this.norm);
  }
}
