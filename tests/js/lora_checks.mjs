// CPU-only checks of the Node host's LoRA module (lora.js): fp16 rounding, the stacked side path,
// key inspection and the loader's name matching against fake models that list their linears.
// Reads a JSON job file, prints one JSON object for tests/test_lora_host.py.
import fs from "fs";
import path from "path";
import { fileURLToPath, pathToFileURL } from "url";

const here = path.dirname(fileURLToPath(import.meta.url));
const js = path.resolve(here, "..", "..", "nanosaur2-web_amd", "js");
const mod = (f) => import(pathToFileURL(path.join(js, f)).href);

async function main() {
  const job = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  const L = await mod("lora.js");
  const out = {};
  out.f16 = Array.from(L.f32ToF16Bits(Float32Array.from(job.f16)));
  const W = { name: "w", N: job.N, K: job.K, lora: job.entries.map((e) => ({ ...e, A: Float32Array.from(e.A), B: Float32Array.from(e.B) })) };
  const s = L.stackLora(W);
  out.stack = { R: s.R, a: Array.from(s.a), b: Array.from(s.b) };
  // a stacked weight whose parts' LoRAs do not fit one side path: cut into windows of whole parts
  const toEntry = (e) => ({ ...e, A: Float32Array.from(e.A), B: Float32Array.from(e.B) });
  const SW = { name: "stacked", N: job.stacked.N, K: job.stacked.K, parts: job.stacked.parts, lora: job.stacked.entries.map(toEntry) };
  out.windows = L.loraWindows(SW).map((w) => {
    const st = L.stackLora(SW, w);
    return { off: w.off, n: w.n, R: st.R, a: Array.from(st.a), b: Array.from(st.b) };
  });
  const big = { ...SW, lora: [toEntry({ ...job.stacked.entries[0], r: 260 })] };
  try {
    L.loraWindows(big);
    out.rankError = null;
  } catch (e) {
    out.rankError = String(e.message);
  }
  out.inspect = job.keys.map((ks) => L.inspectLoraKeys(ks));
  // loaders against fake registries built from { name, kind, N, K } linears (and stacked parts)
  out.loads = [];
  for (const ld of job.loads) {
    const model = { linears: () => ld.linears.map((l) => ({ ...l, buf: {} })) };
    const reg = L.linearRegistry(model);
    const regs = ld.te ? { te: reg } : { dit: reg };
    const res = await L.loadLora(ld.file, regs);
    out.loads.push({
      matched: res.matched, total: res.total, skipped: res.skipped, unsupported: res.unsupported,
      modules: res.modules.map((m) => ({ W: m.target.W.name || m.target.W.parts.map((p) => p.name).join("+"),
        off: m.target.off, n: m.target.n, r: m.r, alphaScale: m.alphaScale, A: Array.from(m.A.slice(0, 512)) })),
    });
  }
  process.stdout.write(JSON.stringify(out) + "\n");
}

main().catch((e) => {
  process.stderr.write(String(e && e.stack ? e.stack : e) + "\n");
  process.exit(1);
});
