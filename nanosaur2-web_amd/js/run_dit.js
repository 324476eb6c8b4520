// Command-line driver for one Nanosaur2 DiT pass on the MI355X through the Node host.
//
//   node run_dit.js (--weights FILE.safetensors | --synthetic SEED)
//                   (--inputs DIR | --shape H,W,T[,SEED])
//                   [--out FILE.f32] [--reference-ops] [--path-drop] [--lora FILE[:STRENGTH]]...
//                   [--warmup N] [--reps N] [--profile] [--abort-at K]
//
// --inputs DIR holds inputs.json {h, w, sigma, T} and latent.f32 [64*h*w], context.f32
// [T*640], weights.f32 [T]. --out writes the x0 prediction [64, h, w] as raw fp32.
// With --reps, the pass is timed with the latent resident in device memory (stream events
// and wall clock), and as many times host-to-host (upload, pass, readback; the median, since a
// lone host hiccup can double one sample); one JSON line with
// the timings (and the per-op profile with --profile) is printed. The passes are timed twice:
// one at a time (each waits for the previous to finish: `ms_device`), and queued (issued back
// to back behind one untimed pass, with no wait between them: `ms_device_queued`), so that a
// pass's launches are on the device before they run, as in a pipelined sampler loop (the host
// issues a pass faster than the GPU runs it); the per-op profile is taken on queued passes, so
// it times the ops' own execution rather than the host's launch latency between them. --lora attaches a LoRA file
// (strength 1 by default; repeatable) to the model's linears (lora.js), as the pipeline does.
// --abort-at K first runs a pass whose onBlock throws an AbortError after block K, as the
// pipeline's cancel does, and reports the error, the blocks run and the pooled bytes in use
// before and after it; the other passes follow on the same model.

import fs from "fs";
import path from "path";
import { GPU } from "./device.js";
import { native } from "./native.js";
import { Nanosaur2DiT } from "./nanosaur2.js";
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
    else if (k === "--inputs") a.inputs = next();
    else if (k === "--shape") a.shape = next().split(",").map(Number);
    else if (k === "--out") a.out = next();
    else if (k === "--reference-ops") a.referenceOps = true;
    else if (k === "--path-drop") a.pathDrop = true;
    else if (k === "--warmup") a.warmup = Number(next());
    else if (k === "--reps") a.reps = Number(next());
    else if (k === "--profile") a.profile = true;
    else if (k === "--lora") a.loras.push(parseLora(next()));
    else if (k === "--abort-at") a.abortAt = Number(next());
    else throw new Error(`unknown argument ${k}`);
  }
  return a;
}

// "FILE[:STRENGTH]" -> { file, strength }
export function parseLora(arg) {
  const m = /^(.*):(-?[\d.]+)$/.exec(arg);
  return m ? { file: m[1], strength: Number(m[2]) } : { file: arg, strength: 1 };
}

function readF32(file) {
  const b = fs.readFileSync(file);
  return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
}

// Seeded inputs of the benchmark shape (values only matter for timing).
function syntheticInputs([h, w, T, seed = 1]) {
  let s = (seed * 2654435761) >>> 0 || 1;
  const u = () => {
    s ^= s << 13; s >>>= 0; s ^= s >>> 17; s ^= s << 5; s >>>= 0;
    return s / 4294967296;
  };
  const gauss = (n) => {
    const o = new Float32Array(n);
    for (let i = 0; i < n; i++) o[i] = Math.sqrt(-2 * Math.log(u() + 1e-12)) * Math.cos(2 * Math.PI * u());
    return o;
  };
  const weights = new Float32Array(T);
  for (let i = 0; i < T; i++) weights[i] = 0.5 + u();
  return { h, w, T, sigma: u(), latent: gauss(64 * h * w), context: gauss(T * 640), weights };
}

function loadInputs(dir) {
  const meta = JSON.parse(fs.readFileSync(path.join(dir, "inputs.json"), "utf8"));
  return {
    h: meta.h, w: meta.w, T: meta.T, sigma: meta.sigma,
    latent: readF32(path.join(dir, "latent.f32")),
    context: readF32(path.join(dir, "context.f32")),
    weights: readF32(path.join(dir, "weights.f32")),
  };
}

const median = (xs) => {
  const s = [...xs].sort((p, q) => p - q);
  return s.length ? s[Math.floor(s.length / 2)] : null;
};

async function main() {
  const a = parseArgs(process.argv.slice(2));
  const t0 = Date.now();
  const gpu = await GPU.create({ profile: !!a.profile });
  const st = a.weights ? await SafeTensors.open(a.weights) : new SyntheticWeights(a.synthetic || 3);
  const dit = await Nanosaur2DiT.load(gpu, st, null, { fused: !a.referenceOps });
  if (st.close) st.close();
  const loraReports = [];
  if (a.loras.length) {
    const regs = { dit: linearRegistry(dit) };
    const active = [];
    for (const { file, strength } of a.loras) {
      const L = await loadLora(file, regs);
      loraReports.push({ file, strength, matched: L.matched, total: L.total, unsupported: L.unsupported, skipped: L.skipped });
      active.push({ lora: L, strength });
    }
    attachLoras(regs, active);
  }
  const inp = a.inputs ? loadInputs(a.inputs) : syntheticInputs(a.shape || [76, 52, 256]);
  const { h, w, sigma } = inp;
  const text = dit.prepareText(inp.context, Array.from(inp.weights));
  const loadMs = Date.now() - t0;
  const report = { h, w, T: inp.T, tokens: h * w, fused: !a.referenceOps, pathDrop: !!a.pathDrop, load_ms: loadMs, device: gpu.info,
    loras: loraReports, weight_bytes: dit.weightBytes() };

  if (a.abortAt !== undefined) {
    // a cancelled pass (app/pipeline.js:233-247 throws from onBlock)
    dit.rope(h, w);  // the RoPE table is cached per shape on first use: not part of the pass
    await gpu.sync();
    const liveBefore = gpu.pool.live;
    let blocks = 0;
    const onBlock = async () => {
      blocks++;
      await gpu.sync();
      if (blocks >= a.abortAt) {
        const e = new Error("Generation cancelled");
        e.name = "AbortError";
        throw e;
      }
    };
    let error = null;
    try {
      await dit.forward(inp.latent, h, w, text, sigma, { pathDrop: !!a.pathDrop, onBlock });
    } catch (e) {
      error = e.name;
    }
    await gpu.sync();
    report.abort = { at: a.abortAt, blocks, error, live_before: liveBefore, live_after: gpu.pool.live };
  }

  if (a.out) {
    const x0 = await dit.forward(inp.latent, h, w, text, sigma, { pathDrop: !!a.pathDrop });
    fs.writeFileSync(a.out, Buffer.from(x0.buffer));
    report.out = a.out;
  }

  if (a.reps > 0) {
    // device-resident latent tokens [L, 64]
    const L = h * w;
    const tok = new Float32Array(L * 64);
    for (let ch = 0; ch < 64; ch++) for (let l = 0; l < L; l++) tok[l * 64 + ch] = inp.latent[ch * L + l];
    const tokens = gpu.fromArray(tok, [L, 64]);
    const pass = async () => (await dit.forwardTokens(tokens, h, w, text, sigma, { pathDrop: !!a.pathDrop })).release();
    for (let i = 0; i < a.warmup; i++) await pass();
    await gpu.sync();
    if (gpu.profiler) gpu.profiler.reset();
    const evs = [];
    for (let i = 0; i < 2 * a.reps; i++) evs.push(native.eventCreate());
    // one pass at a time: each waits for the previous one
    const single = async () => {
      const dev = [];
      const wall = [];
      for (let i = 0; i < a.reps; i++) {
        const w0 = process.hrtime.bigint();
        native.eventRecord(evs[0]);
        await pass();
        native.eventRecord(evs[1]);
        await gpu.sync();
        wall.push(Number(process.hrtime.bigint() - w0) / 1e6);
        dev.push(native.eventElapsed(evs[0], evs[1]));
        process.stderr.write(`[run_dit] pass ${i + 1}/${a.reps}: ${dev[dev.length - 1].toFixed(3)} ms\n`);
      }
      return { dev, wall };
    };
    // queued: one untimed pass, then the timed passes issued back to back, one wait at the end
    const queued = async () => {
      if (gpu.profiler) gpu.profiler.paused = true;
      await pass();
      if (gpu.profiler) gpu.profiler.paused = false;
      for (let i = 0; i < a.reps; i++) {
        native.eventRecord(evs[2 * i]);
        await pass();
        native.eventRecord(evs[2 * i + 1]);
      }
      await gpu.sync();
      const dev = [];
      for (let i = 0; i < a.reps; i++) dev.push(native.eventElapsed(evs[2 * i], evs[2 * i + 1]));
      // the whole run of passes, first start to last end: any gap the host leaves between passes counts
      const total = native.eventElapsed(evs[0], evs[2 * a.reps - 1]);
      process.stderr.write(`[run_dit] queued passes: ${dev.map((d) => d.toFixed(3)).join(" ")} ms; ` +
                           `${a.reps} passes in ${total.toFixed(3)} ms\n`);
      return { devQ: dev, total };
    };
    const { dev, wall } = gpu.profiler ? { dev: [], wall: [] } : await single();
    const { devQ, total } = await queued();
    if (gpu.profiler) {
      const rows = await gpu.profiler.report();
      report.profile = rows.map((r) => ({ name: r.name, count: r.count / a.reps, ms: r.ms / a.reps, tflops: r.flops ? r.flops / (r.ms / 1e3) / 1e12 : null }));
    }
    const host = [];
    for (let i = 0; i < a.reps; i++) {
      const w0 = process.hrtime.bigint();
      await dit.forward(inp.latent, h, w, text, sigma, { pathDrop: !!a.pathDrop });
      host.push(Number(process.hrtime.bigint() - w0) / 1e6);
    }
    tokens.release();
    for (const e of evs) native.eventDestroy(e);
    Object.assign(report, {
      reps: a.reps, warmup: a.warmup, ms_device: dev, ms_wall: wall, ms_host_to_host: host,
      ms_device_median: median(dev), ms_wall_median: median(wall), ms_host_to_host_median: median(host),
      ms_device_queued: devQ, ms_device_queued_median: median(devQ),
      ms_device_queued_total: total, ms_device_queued_per_pass: total / a.reps,
    });
  }
  report.pool_peak_bytes = gpu.pool.peak;
  text.release();
  dit.unload();
  process.stdout.write(JSON.stringify(report) + "\n");
}

main().catch((e) => {
  process.stderr.write(`[run_dit] error: ${e && e.stack ? e.stack : e}\n`);
  process.exit(1);
});
