// Rotary tables for the split-half RoPE convention (pair i is (x[i], x[i + D/2])): a cos block
// followed by a sin block, each [L][D/2], uploaded as one fp32 tensor whose .sinOff marks the
// sin block (the layout of app/models/common.js:1-13, consumed by headNorm and attention).

function upload(gpu, angles, L, half) {
  const n = L * half;
  const cs = new Float32Array(2 * n);
  for (let i = 0; i < n; i++) {
    const a = angles[i];
    cs[i] = Math.cos(a);
    cs[n + i] = Math.sin(a);
  }
  const t = gpu.fromArray(cs, [cs.length]);
  t.sinOff = n;
  return t;
}

// Frequencies 1 / theta^(2i/D), i < D/2, each step rounded to fp32 (app/models/common.js:15).
function frequencies(D, theta) {
  const f = new Float64Array(D / 2);
  for (let i = 0; i < D / 2; i++) f[i] = Math.fround(1 / Math.pow(theta, Math.fround((2 * i) / D)));
  return f;
}

// 1-D RoPE: angle(l, i) = l * f_i (app/models/common.js:17-24).
export function ropeTable(gpu, L, D, theta) {
  const half = D / 2;
  const f = frequencies(D, theta);
  const a = new Float32Array(L * half);
  for (let l = 0; l < L; l++) for (let i = 0; i < half; i++) a[l * half + i] = l * f[i];
  return upload(gpu, a, L, half);
}

// Nanosaur2 2-D RoPE over centred token coordinates (token l = y*W + x): the first D/4 pairs
// rotate by x - (W-1)/2, the next D/4 by y - (H-1)/2, both with the frequencies of a
// D/2-dimensional axis at theta 10000 (app/models/common.js:26-43; tools/reference.py:220-227).
export function rope2dTable(gpu, H, W, D) {
  const half = D / 2;
  const quarter = half / 2;
  const f = frequencies(half, 10000);
  const a = new Float32Array(H * W * half);
  for (let y = 0; y < H; y++) {
    const cy = y - (H - 1) / 2;
    for (let x = 0; x < W; x++) {
      const cx = x - (W - 1) / 2;
      const base = (y * W + x) * half;
      for (let i = 0; i < quarter; i++) {
        a[base + i] = cx * f[i];
        a[base + quarter + i] = cy * f[i];
      }
    }
  }
  return upload(gpu, a, H * W, half);
}
