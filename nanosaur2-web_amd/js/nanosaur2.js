// Nanosaur2 DiT (1536 wide, 18 blocks, 16 heads of 96) on the ns2 ops: one pass from a
// latent [64, h, w] to the x0 prediction, with the composition of the reference's
// Nanosaur2DiT (app/models/nanosaur2.js:38-258; tools/reference.py:248-329):
//   text:   y_embedder (+RMSNorm) -> 2 text-refine blocks conditioned on the timestep;
//           prompt weights pool the refined text and become log-biases on the text keys
//   blocks: adaLN-single modulation (shared projection + per-block offset), QK-norm, 2-D RoPE,
//           joint image+text attention on even blocks (kv_y), image-only on odd blocks,
//           SwiGLU MLP, gated residuals; blocks 2..15 form the SPRINT residual path.
//
// fused (default): normMod and GLU write the rotated fp16 operand of the next int8 linear,
// and the per-head norms and RoPE run inside the attention call. fused = false issues the
// reference's op sequence (separate headNorm / rotate / glu ops) on the same kernels' API.

import * as ops from "./ops.js";
import { rope2dTable } from "./common.js";
import { concatLinears } from "./weights.js";

const D = 1536;
const HEADS = 16;
const HD = D / HEADS;
const BLOCKS = 18;
const SPRINT_F = 2;
const SPRINT_H = 2;
const CH = 64;

// Sinusoidal embedding of sigma * 1000, cos half then sin half, 256 dims, computed in fp32
// steps (app/models/nanosaur2.js:24-36; tools/reference.py:213-217).
// Sinusoidal embedding of t = 1000 sigma: 128 cosines, then 128 sines, of t times the frequencies
// exp(-ln(1e4) i / 128). The frequency table, the product t f and t itself are rounded to fp32
// where the reference rounds them (app/models/nanosaur2.js:25-36), which makes the embedding
// bit-identical to the reference's.
const T_FREQS = Float32Array.from({ length: 128 }, (_, i) => Math.exp(Math.fround((-Math.log(10000) * i) / 128)));

export function timestepEmbedding(sigma) {
  const t = Math.fround(sigma * 1000);
  const n = T_FREQS.length;
  const emb = new Float32Array(2 * n);
  T_FREQS.forEach((f, i) => {
    const angle = Math.fround(t * f);
    emb[i] = Math.cos(angle);
    emb[n + i] = Math.sin(angle);
  });
  return emb;
}

export class Nanosaur2DiT {
  // st: { linear(gpu, base), vector(gpu, name), has(name) } (weights.js SafeTensors)
  static async load(gpu, st, onProgress, { fused = true } = {}) {
    const m = new Nanosaur2DiT(gpu, fused);
    const lin = (n) => st.linear(gpu, n);
    const vec = (n) => st.vector(gpu, n);
    m.sEmbed = await lin("s_embedder.proj.");
    m.t1 = await lin("t_embedder.mlp.0.");
    m.t2 = await lin("t_embedder.mlp.2.");
    m.yEmbed = await lin("y_embedder.proj.");
    m.yNorm = await vec("y_embedder.norm.weight");
    m.yPool = await lin("y_pool_proj.");
    m.sharedAda = await lin("shared_encoder_adaLN.0.");
    m.sprintOut = await lin("sprint_out_proj.");
    m.text = [];
    for (let i = 0; st.has(`text_refine_blocks.${i}.norm1.weight`); i++) {
      const p = `text_refine_blocks.${i}.`;
      m.text.push({
        ada: await lin(p + "adaLN_modulation.0."), n1: await vec(p + "norm1.weight"), n2: await vec(p + "norm2.weight"),
        qkv: await lin(p + "attn.qkv."), qn: await vec(p + "attn.q_norm.weight"), kn: await vec(p + "attn.k_norm.weight"),
        proj: await lin(p + "attn.proj."), w12: await lin(p + "mlp.w12."), w3: await lin(p + "mlp.w3."),
      });
    }
    m.blocks = [];
    for (let i = 0; i < BLOCKS; i++) {
      const p = `blocks.${i}.`;
      m.blocks.push({
        offset: await vec(`encoder_adaLN_offsets.${i}`), n1: await vec(p + "norm1.weight"), n2: await vec(p + "norm2.weight"),
        qkv: await lin(p + "attn.qkv_x."), kvY: st.has(p + "attn.kv_y.weight") ? await lin(p + "attn.kv_y.") : null,
        qn: await vec(p + "attn.q_norm.weight"), kn: await vec(p + "attn.k_norm.weight"),
        proj: await lin(p + "attn.proj."), w12: await lin(p + "mlp.w12."), w3: await lin(p + "mlp.w3."),
      });
      if (onProgress) onProgress((i + 1) / BLOCKS);
    }
    m.finalAda = await lin("final_layer.adaLN_modulation.");
    m.finalLinear = await lin("final_layer.linear.");
    if (fused) {
      // the blocks' adaLN offsets in one [BLOCKS, 6D] tensor, so that every pass forms all the
      // block modulations with one launch
      m.offsets = gpu.empty([BLOCKS, 6 * D]);
      m.blocks.forEach((b, i) => ops.elementwise(gpu, "copy", b.offset, null, ops.rowView(m.offsets, i)));
      // the joint blocks' kv_y projections all take the same rotated text: one stacked weight
      // [sum N, K] whose parts keep the blocks' module names, multiplied once per pass; block b
      // reads its k|v columns at kvSlot * N_b (app/models/nanosaur2.js:168-169, 202)
      const joint = m.blocks.filter((b) => b.kvY);
      if (joint.length && joint.every((b) => b.kvY.kind === "i8" && b.kvY.N === joint[0].kvY.N && b.kvY.K === D)) {
        m.kvAll = concatLinears(gpu, joint.map((b) => b.kvY));
        joint.forEach((b, i) => {
          b.kvSlot = i * b.kvY.N;
          b.kvY = null;
        });
      }
      // the fused producers feed the block linears tiled operands: re-tile their weights once
      if (m.kvAll && ops.tileable(m.kvAll)) {
        ops.tileWeight(gpu, m.kvAll);
        ops.dropRowMajor(m.kvAll);
      }
      // the adaLN projections that share an input run as one GEMV over a stacked weight: the text
      // blocks' (all from the timestep embedding), and the shared and final ones (both from the
      // conditioning vector); the parts keep their module names (LoRA targets)
      const gemv = (Ws) => Ws.length > 1 && Ws.every((W) => W.kind === "bf16" && W.K === Ws[0].K);
      if (gemv(m.text.map((b) => b.ada))) {
        m.textAda = concatLinears(gpu, m.text.map((b) => b.ada));
        m.text.forEach((b, i) => {
          b.adaSlot = m.textAda.parts[i].off;
          b.ada = null;
        });
      }
      if (gemv([m.sharedAda, m.finalAda])) {
        m.condAda = concatLinears(gpu, [m.sharedAda, m.finalAda]);
        m.sharedAda = null;
        m.finalAda = null;
      }
      // the 3952-row bf16 linears (patch embedder, SPRINT projection, final layer) take tiled
      // fp16 operands over their weights re-tiled as fp16
      for (const W of [m.sEmbed, m.sprintOut, m.finalLinear]) {
        if (W && ops.tileablePlain(W)) {
          ops.tileWeight(gpu, W);
          ops.dropRowMajor(W);
        }
      }
      for (const b of m.text.concat(m.blocks)) {
        for (const W of [b.qkv, b.kvY, b.proj, b.w3]) if (W && ops.tileable(W)) ops.tileWeight(gpu, W);
        // the image blocks' MLP runs its first linear fused with the GLU and the rotation for w3;
        // the text blocks' (a few hundred rows: 64 work-groups of the fused launch's 64 x 512
        // tiles) run the plain tiled GEMM over 64 x 128 tiles, then the GLU and rotation
        const text = m.text.includes(b);
        if (!text && b.w12.kind === "i8" && b.w12.N % 512 === 0 && b.w12.K % 256 === 0) ops.tileWeightGlu(gpu, b.w12);
        else if (ops.tileable(b.w12)) ops.tileWeight(gpu, b.w12);
        // the fused path feeds every re-tiled weight tiled operands only: keep one copy (w12's
        // GLU tiles serve only while w3 takes the tiled operand the GLU launch writes)
        for (const W of [b.qkv, b.kvY, b.proj, b.w3]) if (W && W.tbuf) ops.dropRowMajor(W);
        if (b.w12.tbuf || (b.w12.tglu && b.w3.tbuf)) ops.dropRowMajor(b.w12);
      }
    }
    return m;
  }

  // Every linear weight of the model (LoRA targets, lora.js linearRegistry).
  linears() {
    const top = [this.sEmbed, this.t1, this.t2, this.yEmbed, this.yPool, this.sharedAda, this.sprintOut,
      this.finalAda, this.finalLinear, this.condAda, this.textAda];
    const text = this.text.flatMap((b) => [b.ada, b.qkv, b.proj, b.w12, b.w3]);
    const blocks = this.blocks.flatMap((b) => [b.qkv, b.kvY, b.proj, b.w12, b.w3]);
    return top.concat(text, blocks, [this.kvAll]).filter((W) => W);
  }

  // Bytes of device memory the loaded weights hold (every persistent buffer, once).
  weightBytes() {
    const seen = new Set();
    let bytes = 0;
    const walk = (o) => {
      if (!o || typeof o !== "object" || seen.has(o)) return;
      seen.add(o);
      if (typeof o.destroy === "function" && o.ptr !== undefined) {
        if (o.ptr !== null) bytes += o.size;
        return;
      }
      for (const k of Object.keys(o)) if (k !== "gpu" && k !== "ropeCache") walk(o[k]);
    };
    walk(this);
    return bytes;
  }

  constructor(gpu, fused = true) {
    this.gpu = gpu;
    this.fused = fused;
    this.ropeCache = new Map();  // "HxW" -> 2-D RoPE table Tensor (depends on the grid only)
  }

  // 2-D RoPE table of an h x w latent grid, built and uploaded once per grid size.
  rope(h, w) {
    const key = `${h}x${w}`;
    let cs = this.ropeCache.get(key);
    if (!cs) {
      cs = rope2dTable(this.gpu, h, w, HD);
      this.ropeCache.set(key, cs);
    }
    return cs;
  }

  // Release every persistent weight buffer.
  unload() {
    if (this.offsets) this.offsets.release();
    this.offsets = null;
    for (const cs of this.ropeCache.values()) cs.release();
    this.ropeCache.clear();
    const seen = new Set();
    const walk = (o) => {
      if (!o || typeof o !== "object" || seen.has(o)) return;
      seen.add(o);
      if (typeof o.destroy === "function" && o.ptr !== undefined) { o.destroy(); return; }
      for (const k of Object.keys(o)) if (k !== "gpu") walk(o[k]);
    };
    walk(this);
  }

  // ------------------------------------------------------------------ text

  // hidden: Float32Array [L, 640]; weights: per-token prompt weights. Tokens with weight <= 0
  // are masked in the reference (no key, zeroed text row, no pooling contribution), so they
  // are dropped; they still count in the pooling denominator (app/models/nanosaur2.js:94-118).
  // The prompt as the blocks consume it (app/models/nanosaur2.js:97-118): tokens of weight > 0
  // through y_embedder (linear, then RMSNorm) -> { L, y [L, D], pool [L] (their weights),
  // poolScale = 1 / max(1, sum of all weights), bias [L] (log weights, floored at 1e-4) or null
  // when every kept weight is 1 }. Zero-weight tokens are dropped where the reference's dense
  // path masks them; the pooling denominator still counts every weight.
  prepareText(hidden, weights) {
    const gpu = this.gpu;
    let total = 0;
    const rows = [];
    for (let i = 0; i < weights.length; i++) {
      total += weights[i];
      if (weights[i] > 0) rows.push(i);
    }
    const L = rows.length;
    if (L === 0) return { L: 0, release() {} };
    const kept = Float32Array.from(rows, (i) => weights[i]);
    const gathered = new Float32Array(L * 640);
    rows.forEach((src, dst) => gathered.set(hidden.subarray(src * 640, src * 640 + 640), dst * 640));
    const ctx = gpu.fromArray(gathered, [L, 640]);
    const emb = ops.linear(gpu, ctx, this.yEmbed, { name: "dit.y_embed" });
    ctx.release();
    const y = ops.rmsnorm(gpu, emb, this.yNorm, D);
    emb.release();
    const pool = gpu.fromArray(kept, [L]);
    // the log of each weight as given (before its fp32 rounding), then rounded once
    const weighted = kept.some((w) => w !== 1);
    const bias = weighted ? gpu.fromArray(Float32Array.from(rows, (i) => Math.log(Math.max(weights[i], 1e-4))), [L]) : null;
    return {
      L, y, pool, poolScale: 1 / Math.max(1, total), bias,
      release() {
        y.release();
        pool.release();
        if (bias) bias.release();
      },
    };
  }

  // Attention over a packed qkv [Lk, 3D] buffer; fused: per-head norms (and RoPE on the
  // first ropeRows rows) inside the attention call, else the reference's headNorm ops.
  // textKV: the text keys and values outside qkv ({ t, off, ld }, from the stacked kv_y product)
  // vpack: the values of the L image keys, already packed by qkvProj
  attend(qkv, L, Lk, b, { cs = null, textRows = 0, bias = null, textKV = null, vpack = null } = {}) {
    const gpu = this.gpu;
    const common = { q: qkv, k: qkv, v: qkv, Lq: L, Lk, H: HEADS, D: HD, ldq: 3 * D, ldk: 3 * D, ldv: 3 * D,
      qOff: 0, kOff: D, vOff: 2 * D, bias, biasStart: L };
    if (this.fused) {
      return ops.attention(gpu, { ...common, qNorm: b.qn, kNorm: b.kn, cs, ropeRows: L,
        textKV: textKV ? { ...textKV, start: L } : null, vPacked: vpack ? { buf: vpack, rows: L } : null });
    }
    ops.headNorm(gpu, qkv, b.qn, { L, H: HEADS, D: HD, ld: 3 * D, colOff: 0, cs });
    ops.headNorm(gpu, qkv, b.kn, { L, H: HEADS, D: HD, ld: 3 * D, colOff: D, cs });
    if (textRows) ops.headNorm(gpu, qkv, b.kn, { L: textRows, H: HEADS, D: HD, ld: 3 * D, colOff: D, rowOff: L });
    return ops.attention(gpu, common);
  }

  // x += gate_mlp * w3(silu(x1) * x2), [x1 x2] = w12(modulate(norm2(x))) (app/models/nanosaur2.js:142-152)
  mlp(x, b, mod) {
    const gpu = this.gpu;
    if (this.fused && b.w12.tglu && b.w3.tbuf) {
      const nr = ops.normModRotated(gpu, x, mod, 3 * D, 4 * D, D, b.n2, 1e-6, true);
      const gr = ops.linearGluRotated(gpu, nr, b.w12, "silu", "dit.mlp.w12");
      nr.release();
      ops.linear(gpu, null, b.w3, { xr: gr, out: x, resid: true, gate: mod, gOff: 5 * D, name: "dit.mlp.w3" });
      gr.release();
      return;
    }
    if (this.fused) {
      const nr = ops.normModRotated(gpu, x, mod, 3 * D, 4 * D, D, b.n2, 1e-6, !!b.w12.tbuf);
      const h = ops.linear(gpu, null, b.w12, { xr: nr, name: "dit.mlp.w12" });
      nr.release();
      const gr = ops.gluRotated(gpu, h, "silu", !!b.w3.tbuf);
      h.release();
      ops.linear(gpu, null, b.w3, { xr: gr, out: x, resid: true, gate: mod, gOff: 5 * D, name: "dit.mlp.w3" });
      gr.release();
      return;
    }
    const n = ops.normMod(gpu, x, mod, 3 * D, 4 * D, D, b.n2);
    const h = ops.linear(gpu, n, b.w12, { name: "dit.mlp.w12" });
    n.release();
    const g = ops.glu(gpu, h, "silu");
    h.release();
    ops.linear(gpu, g, b.w3, { out: x, resid: true, gate: mod, gOff: 5 * D, name: "dit.mlp.w3" });
    g.release();
  }

  // x += gate_msa * proj(a); fused: a is rotated into the tiled operand of the int8 GEMM
  projAdd(x, a, W, mod, name) {
    const gpu = this.gpu;
    if (this.fused && W.tbuf) {
      const ar = ops.rotateHalf(gpu, a, D, true);
      ops.linear(gpu, null, W, { xr: ar, out: x, resid: true, gate: mod, gOff: 2 * D, name });
      ar.release();
      return;
    }
    ops.linear(gpu, a, W, { out: x, resid: true, gate: mod, gOff: 2 * D, name });
  }

  // qkv projection of modulate(norm1(x)) into rows [0, L) of qkv; vpack: the values go into
  // this packedValues() tensor instead of qkv's v columns (tiled weights only)
  qkvProj(x, mod, b, qkv, name, vpack = null) {
    const gpu = this.gpu;
    if (this.fused) {
      const nr = ops.normModRotated(gpu, x, mod, 0, D, D, b.n1, 1e-6, !!b.qkv.tbuf);
      ops.linear(gpu, null, b.qkv, { xr: nr, out: qkv, name, vpack: vpack ? { buf: vpack, col0: 2 * D } : null });
      nr.release();
      return;
    }
    const n = ops.normMod(gpu, x, mod, 0, D, D, b.n1);
    ops.linear(gpu, n, b.qkv, { out: qkv, name });
    n.release();
  }

  // Text refine blocks for one timestep: Tensor [L, D] (app/models/nanosaur2.js:120-140)
  refineText(text, tc) {
    const gpu = this.gpu;
    const L = text.L;
    const txt = ops.elementwise(gpu, "copy", text.y);
    // every text block's modulation at once from the stacked adaLN weight
    const mods = this.textAda ? ops.linear(gpu, tc, this.textAda, { name: "dit.text.ada" }) : null;
    for (const b of this.text) {
      const mod = mods ? ops.colView(mods, b.adaSlot, 6 * D) : ops.linear(gpu, tc, b.ada, { name: "dit.text.ada" });
      const qkv = gpu.empty([L, 3 * D]);
      this.qkvProj(txt, mod, b, qkv, "dit.text.qkv");
      const a = this.attend(qkv, L, L, b);
      qkv.release();
      this.projAdd(txt, a, b.proj, mod, "dit.text.proj");
      a.release();
      this.mlp(txt, b, mod);
      mod.release();
    }
    if (mods) mods.release();
    return txt;
  }

  // ------------------------------------------------------------------ conditioning

  // Everything that depends on sigma and the prompt but not on the latent
  // (app/models/nanosaur2.js:154-184).
  condition(text, sigma) {
    const gpu = this.gpu;
    const temb = gpu.fromArray(timestepEmbedding(sigma), [1, 256]);
    const h = ops.linear(gpu, temb, this.t1, { act: "silu", name: "dit.t_embed" });
    temb.release();
    const t = ops.linear(gpu, h, this.t2, { name: "dit.t_embed" });
    h.release();
    const tc = ops.elementwise(gpu, "silu", t);
    let txt = null;
    let txtR = null;
    let kvText = null;
    if (text.L) {
      txt = this.refineText(text, tc);
      // the int8 kv_y projections take rotated inputs: rotate the text once for all blocks;
      // with the stacked weight, project it for every joint block at once
      if (this.kvAll) {
        txtR = ops.rotateHalf(gpu, txt, D, !!this.kvAll.tbuf);
        kvText = ops.linear(gpu, null, this.kvAll, { xr: txtR, name: "dit.kv_y" });
        txtR.release();
        txtR = null;
      } else if (this.blocks.some((b) => b.kvY && ops.needsRotation(b.kvY))) {
        const tiled = this.blocks.every((b) => !b.kvY || b.kvY.tbuf);
        txtR = this.fused ? ops.rotateHalf(gpu, txt, D, tiled) : ops.rotate(gpu, txt);
      }
      const pooled = ops.rowSum(gpu, txt, text.pool, text.poolScale);
      ops.linear(gpu, pooled, this.yPool, { out: t, resid: true, name: "dit.y_pool" });
      pooled.release();
    }
    tc.release();
    const cond = ops.elementwise(gpu, "silu", t);
    t.release();
    // the shared block modulation and the final layer's, from one stacked GEMV when stacked
    const ada = this.condAda ? ops.linear(gpu, cond, this.condAda, { name: "dit.shared_ada" }) : null;
    const mod = ada ? ops.colView(ada, 0, 6 * D) : ops.linear(gpu, cond, this.sharedAda, { name: "dit.shared_ada" });
    const final = ada ? ops.colView(ada, 6 * D, 2 * D) : ops.linear(gpu, cond, this.finalAda, { name: "dit.final_ada" });
    cond.release();
    // every block's modulation mod + offset_i (app/models/nanosaur2.js:190) at once
    const modAll = this.offsets ? ops.addRows(gpu, mod, this.offsets) : null;
    return {
      txt, txtR, kvText, mod, final, modAll,
      release() {
        if (txt) txt.release();
        if (txtR) txtR.release();
        if (kvText) kvText.release();
        mod.release();
        final.release();
        if (ada) ada.release();
        if (modAll) modAll.release();
      },
    };
  }

  // ------------------------------------------------------------------ forward

  // One DiT block in place on x [L, D] (app/models/nanosaur2.js:186-214).
  block(i, x, L, text, c, cs) {
    const gpu = this.gpu;
    const b = this.blocks[i];
    const mod = c.modAll ? ops.rowView(c.modAll, i) : ops.elementwise(gpu, "add", c.mod, b.offset); // [1, 6D]
    const stacked = b.kvSlot !== undefined && !!c.kvText;
    const cross = !!((b.kvY || stacked) && text.L);
    // rows [0, L): image q|k|v; rows [L, L + text): text k|v (q columns unused), unless the
    // text k|v come from the stacked kv_y product
    const Lk = L + (cross ? text.L : 0);
    const qkv = gpu.empty([stacked ? L : Lk, 3 * D]);
    // fused path: the qkv GEMM writes the image values straight into the attention's fp16 layout
    // (the same rounding the attention's operand pack applies), 16-key groups at a time
    const vpack = this.fused && b.qkv.tbuf && L % 16 === 0 ? ops.packedValues(gpu, Lk, HEADS, HD) : null;
    this.qkvProj(x, mod, b, qkv, "dit.qkv", vpack);
    if (cross && !stacked) {
      ops.linear(gpu, c.txt, b.kvY, { xr: c.txtR, out: qkv, ldc: 3 * D, cOff: L * 3 * D + D, name: "dit.kv_y" });
    }
    const textKV = cross && stacked ? { t: c.kvText, off: b.kvSlot, ld: this.kvAll.N } : null;
    const a = this.attend(qkv, L, Lk, b, { cs, textRows: cross ? text.L : 0, bias: cross ? text.bias : null, textKV,
      vpack });
    qkv.release();
    if (vpack) vpack.release();
    this.projAdd(x, a, b.proj, mod, "dit.proj");
    a.release();
    this.mlp(x, b, mod);
    mod.release();
  }

  // Device-resident pass: tokens [L, 64] (Tensor) -> out [L, 64] (Tensor, caller releases).
  // onBlock(fraction done) is awaited after every block; the pipeline cancels a generation by
  // throwing from it (app/pipeline.js:233-247). An error from a block or from onBlock ends the
  // pass: its tensors go back to the pool before the error propagates, so the model stays
  // usable (work already queued on the stream finishes before the buffers are reused).
  async forwardTokens(tokens, h, w, text, sigma, { pathDrop = false, onBlock } = {}) {
    const gpu = this.gpu;
    const L = h * w;
    let x;
    if (this.sEmbed.tbuf) {
      const tt = ops.toTiled(gpu, tokens);
      x = ops.linear(gpu, null, this.sEmbed, { xr: tt, name: "dit.s_embed" });
      tt.release();
    } else {
      x = ops.linear(gpu, tokens, this.sEmbed, { name: "dit.s_embed" });
    }
    const cs = this.rope(h, w);
    let c = null;
    let g = null;
    try {
      c = this.condition(text, sigma);
      const total = pathDrop ? SPRINT_F + SPRINT_H : BLOCKS;
      let done = 0;
      const run = async (i, s) => {
        this.block(i, s, L, text, c, cs);
        if (onBlock) await onBlock(++done / total);
      };
      for (let i = 0; i < SPRINT_F; i++) await run(i, x);
      if (!pathDrop) {
        g = ops.elementwise(gpu, "copy", x);
        for (let i = SPRINT_F; i < BLOCKS - SPRINT_H; i++) await run(i, g);
        // x += (g - x) W^T; with the tiled weight the difference is formed as its fp16 operand
        const tiled = !!this.sprintOut.tbuf;
        const d = tiled ? ops.toTiled(gpu, g, x) : ops.elementwise(gpu, "sub", g, x);
        g.release();
        g = null;
        ops.linear(gpu, tiled ? null : d, this.sprintOut, { xr: tiled ? d : undefined, out: x, resid: true,
          name: "dit.sprint_out" });
        d.release();
      }
      for (let i = BLOCKS - SPRINT_H; i < BLOCKS; i++) await run(i, x);
    } catch (e) {
      if (g) g.release();
      if (c) c.release();
      x.release();
      throw e;
    }
    const tiled = !!this.finalLinear.tbuf;
    const n = tiled ? ops.normModTiled(gpu, x, c.final, 0, D, D) : ops.normMod(gpu, x, c.final, 0, D, D);
    x.release();
    c.release();
    const out = ops.linear(gpu, tiled ? null : n, this.finalLinear, { xr: tiled ? n : undefined, name: "dit.final" });
    n.release();
    return out;
  }

  // latent: Float32Array [64, h, w]; text: prepareText(...). Returns x0 [64, h, w]
  // (app/models/nanosaur2.js:216-258).
  // The latent <-> token transposes run on the device (the reference does them in JS loops,
  // app/models/nanosaur2.js:220-221, 254-255: ~4.6 ms per pass at 832x1216 on the host).
  async forward(latent, h, w, text, sigma, opts = {}) {
    const gpu = this.gpu;
    const L = h * w;
    const lat = gpu.fromArray(latent, [CH, L]);
    const xin = ops.transpose(gpu, lat); // [L, 64]
    lat.release();
    let out;
    try {
      out = await this.forwardTokens(xin, h, w, text, sigma, opts);
    } finally {
      xin.release();
    }
    const x0t = ops.transpose(gpu, out); // [64, L]
    out.release();
    const x0 = await gpu.read(x0t);
    x0t.release();
    return x0;
  }
}
