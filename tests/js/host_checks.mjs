// CPU-only checks of the Node host (no GPU): module loading, the addon's exports and error
// path, the rotary tables and timestep embedding, and the safetensors reader, using a fake
// device object that captures uploads. Prints one JSON object for tests/test_abi.py.
import path from "path";
import { fileURLToPath, pathToFileURL } from "url";

const here = path.dirname(fileURLToPath(import.meta.url));
const js = path.resolve(here, "..", "..", "nanosaur2-web_amd", "js");
const mod = (f) => import(pathToFileURL(path.join(js, f)).href);

async function main() {
  const out = {};
  const { native } = await mod("native.js");
  out.addonExports = Object.keys(native).sort();
  out.poolRound = [1, 256, 257, 1000, 4096, 5000, 1 << 20, (1 << 20) + 1].map((b) => native.poolRound(b));
  try {
    native.init(0);
    out.initError = null;
  } catch (e) {
    out.initError = String(e.message);
  }
  try {
    native.linearI8(null, 0, 256, null, null, null, null, null, 1, 1, 256, 1, 0, 1, 0, 0, null, 0);
    out.callError = null;
  } catch (e) {
    out.callError = String(e.message);
  }
  try {
    native.hadamard256(5, 0n, 1);
    out.typeError = null;
  } catch (e) {
    out.typeError = String(e.message);
  }

  // fake device: fromArray keeps the host array
  const fake = {
    uploads: [],
    fromArray(arr, shape) { return { arr: Float32Array.from(arr), shape, release() {} }; },
    upload(arr) { this.uploads.push(arr); return { ptr: 1n, size: arr.byteLength, destroy() {} }; },
  };
  const { rope2dTable, ropeTable } = await mod("common.js");
  const t = rope2dTable(fake, 5, 7, 96);
  out.rope2d = { sinOff: t.sinOff, values: Array.from(t.arr) };
  const r1 = ropeTable(fake, 4, 8, 10000);
  out.rope1d = { sinOff: r1.sinOff, values: Array.from(r1.arr) };
  // bounds of host <-> device copies: every error is raised before the addon is called, so a
  // GPU object without a device (and fake buffers) exercises them
  const { GPU, DeviceBuffer, Tensor } = await mod("device.js");
  const g = new GPU({});
  const bounds = {};
  const tryMsg = (f) => { try { f(); return null; } catch (e) { return String(e.message); } };
  bounds.writeOverrun = tryMsg(() => g.write(new DeviceBuffer(1n, 16), new Float32Array(5)));
  bounds.writeOffset = tryMsg(() => g.write(new DeviceBuffer(1n, 16), new Float32Array(4), 4));
  bounds.writeReleased = tryMsg(() => g.write(new DeviceBuffer(null, 16), new Float32Array(1)));
  bounds.fromArrayShape = tryMsg(() => g.fromArray(new Float32Array(7), [2, 3]));
  bounds.readCount = await g.read(new Tensor(g, new DeviceBuffer(1n, 256, true), [2, 3], 256), 7)
    .then(() => null, (e) => String(e.message));
  out.bounds = bounds;
  const { timestepEmbedding } = await mod("nanosaur2.js");
  out.temb = Array.from(timestepEmbedding(0.37));

  const file = process.argv[2];
  if (file) {
    const { SafeTensors } = await mod("weights.js");
    const st = await SafeTensors.open(file);
    const lin = await st.linear(fake, "blk.qkv.");
    const bf = await st.linear(fake, "emb.");
    const vec = await st.f32("norm.weight");
    out.st = {
      i8: { kind: lin.kind, N: lin.N, K: lin.K, bytes: fake.uploads[0].byteLength, scaleLen: lin.scale.size / 4,
        first: Array.from(new Int8Array(fake.uploads[0].buffer, fake.uploads[0].byteOffset, 8)) },
      bf16: { kind: bf.kind, N: bf.N, K: bf.K },
      vec: Array.from(vec),
    };
    try {
      await st.linear(fake, "bad.");
      out.st.badError = null;
    } catch (e) {
      out.st.badError = String(e.message);
    }
  }
  process.stdout.write(JSON.stringify(out) + "\n");
}

main().catch((e) => {
  process.stderr.write(String(e && e.stack ? e.stack : e) + "\n");
  process.exit(1);
});
