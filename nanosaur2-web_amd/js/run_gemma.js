// Command-line driver for the Gemma3 text encoder on the MI355X through the Node host.
//
//   node run_gemma.js (--weights FILE.safetensors | --synthetic SEED)
//                     (--ids FILE.json | --tokens N[,SEED])
//                     [--out FILE.f32] [--warmup N] [--reps N] [--profile] [--lora FILE[:STRENGTH]]...
//                     [--graph] [--graph-check N]
//
// --ids holds a JSON array of token ids; --tokens draws N seeded ids. --out writes the hidden
// states [L, 640] as raw fp32. With --reps the encoder is timed on device-resident embeddings
// (stream events and wall clock); one JSON line with the timings (and the per-op profile with
// --profile) is printed. --graph records one encode as a HIP graph and times (and writes --out
// from) its replays instead. --graph-check N replays the graph N times, alternating the
// embeddings of the ids and of a second seeded id set, with an eager encode between replays,
// and reports each replay's largest difference from the eager encode of the same ids.

import fs from "fs";
import { GPU } from "./device.js";
import { native } from "./native.js";
import * as ops from "./ops.js";
import { Gemma3 } from "./gemma3.js";
import { SafeTensors } from "./weights.js";
import { SyntheticWeights } from "./synthetic.js";
import { linearRegistry, loadLora, attachLoras } from "./lora.js";

function parseArgs(argv) {
  const a = { warmup: 0, reps: 0, loras: [] };
  for (let i = 0; i < argv.length; i++) {
    const k = argv[i];
    const next = () => argv[++i];
    if (k === "--weights") a.weights = next();
    else if (k === "--synthetic") a.synthetic = Number(next());
    else if (k === "--ids") a.ids = JSON.parse(fs.readFileSync(next(), "utf8"));
    else if (k === "--tokens") a.tokens = next().split(",").map(Number);
    else if (k === "--out") a.out = next();
    else if (k === "--warmup") a.warmup = Number(next());
    else if (k === "--reps") a.reps = Number(next());
    else if (k === "--profile") a.profile = true;
    else if (k === "--graph") a.graph = true;
    else if (k === "--graph-check") a.graphCheck = Number(next());
    else if (k === "--lora") {
      const m = /^(.*):(-?[\d.]+)$/.exec(next() || "");
      a.loras.push(m ? { file: m[1], strength: Number(m[2]) } : { file: argv[i], strength: 1 });
    } else throw new Error(`unknown argument ${k}`);
  }
  return a;
}

function seededIds([n, seed = 1], vocab) {
  let s = (seed * 2654435761) >>> 0 || 1;
  const ids = [];
  for (let i = 0; i < n; i++) {
    s ^= s << 13; s >>>= 0; s ^= s >>> 17; s ^= s << 5; s >>>= 0;
    ids.push(s % vocab);
  }
  return ids;
}

const median = (xs) => {
  const s = [...xs].sort((p, q) => p - q);
  return s.length ? s[Math.floor(s.length / 2)] : null;
};

async function main() {
  const a = parseArgs(process.argv.slice(2));
  const t0 = Date.now();
  const gpu = await GPU.create({ profile: !!a.profile });
  const st = a.weights ? await SafeTensors.open(a.weights) : new SyntheticWeights(a.synthetic || 3, { gemma: true });
  const te = await Gemma3.load(gpu, st);
  const loraReports = [];
  if (a.loras.length) {
    const regs = { te: linearRegistry(te) };
    const active = [];
    for (const { file, strength } of a.loras) {
      const L = await loadLora(file, regs);
      loraReports.push({ file, strength, matched: L.matched, total: L.total, unsupported: L.unsupported, skipped: L.skipped });
      active.push({ lora: L, strength });
    }
    attachLoras(regs, active);
  }
  const vocab = (st.info ? st.info("model.embed_tokens.weight") : st.spec.get("model.embed_tokens.weight")).shape[0];
  const ids = a.ids || seededIds(a.tokens || [256, 1], vocab);
  const rows = await st.rows("model.embed_tokens.weight", ids);
  const report = { tokens: ids.length, load_ms: Date.now() - t0, device: gpu.info, loras: loraReports };
  const L = ids.length;
  const graph = a.graph || a.graphCheck ? te.captureEncode(L) : null;
  if (graph) report.graph = true;
  // one graph replay on the embeddings emb (device tensor [L, 640])
  const replay = (emb) => {
    ops.elementwise(gpu, "copy", emb, null, graph.input);
    graph.launch();
  };

  if (a.out) {
    let out;
    if (graph) {
      const emb = te.embed(rows, L);
      replay(emb);
      emb.release();
      out = await gpu.read(graph.output);
    } else {
      const h = te.encodeEmbedded(te.embed(rows, L));
      out = await gpu.read(h);
      h.release();
    }
    fs.writeFileSync(a.out, Buffer.from(out.buffer));
    report.out = a.out;
  }
  if (a.graphCheck) {
    const ids2 = seededIds([L, 7], vocab);
    const embs = [te.embed(rows, L), te.embed(await st.rows("model.embed_tokens.weight", ids2), L)];
    const eager = async (emb) => {
      const h = te.encodeEmbedded(ops.elementwise(gpu, "copy", emb));
      const r = await gpu.read(h);
      h.release();
      return r;
    };
    const refs = [await eager(embs[0]), await eager(embs[1])];
    report.graph_check = [];
    for (let r = 0; r < a.graphCheck; r++) {
      const which = r % 2;
      replay(embs[which]);
      const got = await gpu.read(graph.output);
      await eager(embs[1 - which]); // eager work between replays, on the same pooled buffers
      let d = 0;
      for (let i = 0; i < got.length; i++) d = Math.max(d, Math.abs(got[i] - refs[which][i]));
      report.graph_check.push({ ids: which, max_abs_diff: d });
    }
    for (const e of embs) e.release();
  }
  if (a.reps > 0) {
    const emb = te.embed(rows, L);
    // each pass starts from a copy of the embeddings (the stack updates its input in place)
    // (a graph replay leaves its input intact, so the embeddings are copied in once)
    if (graph) ops.elementwise(gpu, "copy", emb, null, graph.input);
    const pass = graph ? () => graph.launch() : () => te.encodeEmbedded(ops.elementwise(gpu, "copy", emb)).release();
    for (let i = 0; i < a.warmup; i++) pass();
    await gpu.sync();
    if (gpu.profiler) gpu.profiler.reset();
    const evA = native.eventCreate();
    const evB = native.eventCreate();
    const dev = [];
    const wall = [];
    for (let i = 0; i < a.reps; i++) {
      const w0 = process.hrtime.bigint();
      native.eventRecord(evA);
      pass();
      native.eventRecord(evB);
      await gpu.sync();
      wall.push(Number(process.hrtime.bigint() - w0) / 1e6);
      dev.push(native.eventElapsed(evA, evB));
    }
    if (gpu.profiler) {
      const prof = await gpu.profiler.report();
      report.profile = prof.map((r) => ({ name: r.name, count: r.count / a.reps, ms: r.ms / a.reps, tflops: r.flops ? r.flops / (r.ms / 1e3) / 1e12 : null }));
    }
    emb.release();
    native.eventDestroy(evA);
    native.eventDestroy(evB);
    Object.assign(report, { reps: a.reps, warmup: a.warmup, ms_device: dev, ms_wall: wall,
      ms_device_median: median(dev), ms_wall_median: median(wall) });
  }
  if (graph) graph.destroy();
  if (st.close) st.close();
  te.unload();
  process.stdout.write(JSON.stringify(report) + "\n");
}

main().catch((e) => {
  process.stderr.write(`[run_gemma] error: ${e && e.stack ? e.stack : e}\n`);
  process.exit(1);
});
