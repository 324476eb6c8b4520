// Row kernels of the DiT pass: ConvRot rotation (FWHT), normMod, headNorm (+RoPE), GLU,
// elementwise, rowSum and RMSNorm. All are HBM-bound; each reads and writes its row once.
// Fused variants write the rotated fp16 operand of the int8 GEMM directly, so the
// standalone rotation pass of app/gpu/ops.js:38-44 never touches HBM on the DiT path.
#include "ns2_common.h"

using namespace ns2dev;

namespace {

// Store 4 consecutive rotated values (k..k+3, k % 4 == 0) as fp16, row-major or tiled.
__device__ __forceinline__ void store4_f16(uint16_t* __restrict__ y, long long m, int k, int ldy, int K,
                                           int tiled, const float v[4]) {
  uint2 o;
  o.x = pack_half2(v[0], v[1]);
  o.y = pack_half2(v[2], v[3]);
  const long long off = tiled ? tiled_off(m, k, K) : m * ldy + k;
  *reinterpret_cast<uint2*>(y + off) = o;
}

// ---- rotation ------------------------------------------------------------------------------

// y = x H per contiguous 256-group (kernels.js:378-407). One wave per group.
__global__ __launch_bounds__(256) void hadamard256_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y,
                                                           long long groups) {
  long long g = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= groups) return;
  const int lane = threadIdx.x & 63;
  const float4 in = *reinterpret_cast<const float4*>(x + g * 256 + lane * 4);
  float v[4] = {in.x, in.y, in.z, in.w};
  fwht256_wave(v);
  *reinterpret_cast<float4*>(y + g * 256 + lane * 4) = make_float4(v[0], v[1], v[2], v[3]);
}

// Strided [rows, cols] fp32 -> rotated fp16. One wave per 256-group.
__global__ __launch_bounds__(256) void rotate_f16_kernel(const float* __restrict__ x, int ldx,
                                                          uint16_t* __restrict__ y, int ldy,
                                                          int rows, int gpr, int tiled) {
  long long g = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= (long long)rows * gpr) return;
  const int r = (int)(g / gpr), c = (int)(g % gpr) * 256;
  const int lane = threadIdx.x & 63;
  const float4 in = *reinterpret_cast<const float4*>(x + (long long)r * ldx + c + lane * 4);
  float v[4] = {in.x, in.y, in.z, in.w};
  fwht256_wave(v);
  store4_f16(y, r, c + lane * 4, ldy, gpr * 256, tiled, v);
}

// ---- normMod ----------------------------------------------------------------------------

// Reference-layout normMod, any cols (kernels.js:82-117): 256 threads per row.
__global__ __launch_bounds__(256) void norm_mod_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ mod,
                                                        long long shiftOff, long long scaleOff,
                                                        int cols, const float* __restrict__ w,
                                                        float eps, float* __restrict__ y) {
  __shared__ float red[16];
  const long long base = (long long)blockIdx.x * cols;
  float mean = 0.f;
  if (!w) {
    float s = 0.f;
    for (int c = threadIdx.x; c < cols; c += 256) s += x[base + c];
    mean = block_sum(s, red) / (float)cols;
  }
  float v = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    float d = x[base + c] - mean;
    v += d * d;
  }
  const float r = rsqrtf(block_sum(v, red) / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += 256) {
    float n = (x[base + c] - mean) * r;
    if (w) n *= w[c];
    y[base + c] = n * (1.0f + mod[scaleOff + c]) + mod[shiftOff + c];
  }
}

// The same for rows of 256 G columns on 16-byte aligned buffers: one wave per row, 8 rows per
// block, every load of the row issued before any arithmetic (lane l holds columns 4l..4l+3 of
// each 256-column group), the statistics as wave reductions, the same per-element order.
template <int G>
__global__ __launch_bounds__(512) void norm_mod_rows_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ mod,
                                                             long long shiftOff, long long scaleOff, int rows,
                                                             const float* __restrict__ w, float eps,
                                                             float* __restrict__ y) {
  const int row = blockIdx.x * 8 + (threadIdx.x >> 6);
  if (row >= rows) return;
  constexpr int cols = 256 * G;
  const int lane = threadIdx.x & 63;
  const float* src = x + (long long)row * cols + 4 * lane;
  float4 v[G];
#pragma unroll
  for (int g = 0; g < G; ++g) v[g] = *reinterpret_cast<const float4*>(src + 256 * g);
  float mean = 0.f;
  if (!w) {
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) s += (v[g].x + v[g].y) + (v[g].z + v[g].w);
    mean = wave_sum(s) / (float)cols;
  }
  float ss = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    v[g].x -= mean, v[g].y -= mean, v[g].z -= mean, v[g].w -= mean;
    ss += v[g].x * v[g].x + v[g].y * v[g].y + v[g].z * v[g].z + v[g].w * v[g].w;
  }
  const float r = rsqrtf(wave_sum(ss) / (float)cols + eps);
  float* dst = y + (long long)row * cols + 4 * lane;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int c = 256 * g + 4 * lane;
    const float4 sc = *reinterpret_cast<const float4*>(mod + scaleOff + c);
    const float4 sh = *reinterpret_cast<const float4*>(mod + shiftOff + c);
    float4 n = make_float4(v[g].x * r, v[g].y * r, v[g].z * r, v[g].w * r);
    if (w) {
      const float4 ww = *reinterpret_cast<const float4*>(w + c);
      n.x *= ww.x, n.y *= ww.y, n.z *= ww.z, n.w *= ww.w;
    }
    *reinterpret_cast<float4*>(dst + 256 * g) =
        make_float4(n.x * (1.0f + sc.x) + sh.x, n.y * (1.0f + sc.y) + sh.y, n.z * (1.0f + sc.z) + sh.z,
                    n.w * (1.0f + sc.w) + sh.w);
  }
}

// ---- rotated fp16 producers, one wave per row ------------------------------------------------

struct RotRowsArgs {
  const float* x;
  int ldx;
  const float* mod;  // normMod only: shift at mod + shiftOff, scale at mod + scaleOff
  long long shiftOff, scaleOff;
  const float* w;    // normMod only: RMSNorm weight, or null for LayerNorm without affine
  float eps;
  uint16_t* y;
  int ldy, rows, tiled;
};

// [rows, 256 G] fp32 -> (normMod ->) rotated fp16, 8 rows per block
// (ROT false: the fp16 operand of a plain fp16-weight linear, not rotated).
// Each lane loads its 4 values of every group before any arithmetic (the whole row is in
// flight at once), the row statistics are wave reductions, and the 8 rows of a block fill
// whole 128-byte lines of the tiled layout (rows 8q..8q+7 of a k-chunk are adjacent 16-byte
// slots), so no line is assembled from partial writes of different L2s.
// normMod: the block stages the modulation vectors (1 + scale, shift and the norm weight, if
// any) in LDS once, in lane order (slot 64g + l holds the 4 columns lane l uses in group g, so
// the waves' 16-byte reads are conflict-free), instead of every row's wave loading them from
// L1: at 8 rows per block that is 3x the row's own bytes through L1 otherwise. Rows of an even
// number of groups from 4 on take two waves each (16 waves per block), each wave half of the
// row's groups, the two halves' sums added through LDS: twice the waves in flight and half the
// per-wave chain of rotations.
template <int G, bool NORM>
constexpr bool rot_two_waves() { return NORM && G >= 4 && G % 2 == 0; }
template <int G, bool NORM>
constexpr int rot_threads() { return rot_two_waves<G, NORM>() ? 1024 : 512; }

template <int G, bool NORM, bool ROT = true>
__global__ __launch_bounds__((rot_threads<G, NORM>())) void rot_rows_kernel(RotRowsArgs a) {
  constexpr bool WS = rot_two_waves<G, NORM>();
  constexpr int WPR = WS ? 2 : 1;  // waves per row
  // rotation only, rows of an even number of groups from 6 on: each block takes half of its 8
  // rows' groups (the two halves rotate independently), so the grid has twice the blocks and
  // each block stages its whole part in LDS (2432 x 1536: 5.2 -> 4.7 us)
  constexpr int PARTS = (!NORM && G >= 6 && G % 2 == 0) ? 2 : 1;  // column parts per block
  constexpr int GBLK = G / PARTS;                                  // groups of a row per block
  constexpr int GB = GBLK / WPR;                                   // groups per wave
  static_assert(G % (PARTS * WPR) == 0 && GBLK <= 16, "groups per block");
  const int part = PARTS > 1 ? blockIdx.x % PARTS : 0;
  const int wave = threadIdx.x >> 6, rl = wave / WPR;
  const int half = WS ? wave % WPR : 0;  // this wave's half of the block's groups
  const int row = (blockIdx.x / PARTS) * 8 + rl;
  const int gb0 = half * GB;             // the wave's first group within the block's part
  constexpr int cols = 256 * G;
  constexpr int NV = NORM ? 3 : 1;
  __shared__ __attribute__((aligned(16))) float4 mods[NV][NORM ? G * 64 : 1];  // [1 + scale, shift, w]
  // Tiled output goes through LDS (fp16, rows padded by 32 bytes: the 16 units of a quarter-wave
  // write-out read, 2 chunks x 8 rows, fall in 16 different bank groups), at most 16 groups
  // (66 KB), so every 128-byte line of the tiled layout is written whole (direct stores of
  // 6144-column rows wrote each line in 8 pieces: 26.4 us at 2432 rows, 15.1 us staged in two
  // column parts). A wave past the last row still takes part in the block's barriers: it works
  // on the last row, and its result is not written.
  constexpr int TROW = 256 * GBLK + 16;
  __shared__ __attribute__((aligned(16))) uint16_t tout[8 * TROW];
  const bool active = row < a.rows;
  // lane l holds elements 16(l%16) + 4(l/16) .. +3 of every group: the layout of the
  // matrix-core FWHT (its float4 loads still cover each group's 1 KB once per wave). The row's
  // loads are issued first, so that they are in flight while the block stages the modulation
  // (a barrier waits for LDS operations only; a wave past the last row loads the last row).
  const int lane = threadIdx.x & 63;
  const int lo = fwht_mfma_offset();
  const float* src = a.x + (long long)(active ? row : a.rows - 1) * a.ldx + (part * GBLK + gb0) * 256 + lo;
  float v[GB][4];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const float4 in = *reinterpret_cast<const float4*>(src + g * 256);
    v[g][0] = in.x, v[g][1] = in.y, v[g][2] = in.z, v[g][3] = in.w;
  }
  if (NORM) {
    for (int i = threadIdx.x; i < G * 64; i += rot_threads<G, NORM>()) {
      const int c = (i / 64) * 256 + 16 * (i % 16) + 4 * ((i % 64) / 16);
      // the three loads go out together (one wait for all)
      const float4 sc = *reinterpret_cast<const float4*>(a.mod + a.scaleOff + c);
      const float4 sh = *reinterpret_cast<const float4*>(a.mod + a.shiftOff + c);
      const float4 ww = a.w ? *reinterpret_cast<const float4*>(a.w + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      mods[0][i] = make_float4(1.0f + sc.x, 1.0f + sc.y, 1.0f + sc.z, 1.0f + sc.w);
      mods[1][i] = sh;
      if (a.w) mods[NV - 1][i] = ww;
    }
    __syncthreads();
  }
  // with two waves per row every wave reaches the barriers below
  if (!WS && !active && !a.tiled) return;
  float r = 1.f;
  if (NORM) {
    // the two halves' sums of a row meet in LDS (separate slots for the two sums, so no
    // barrier is needed between reading the first and writing the second)
    __shared__ float red[2][8][WPR];
    float mean = 0.f;
    if (!a.w) {
      float s = 0.f;
#pragma unroll
      for (int g = 0; g < GB; ++g) s += (v[g][0] + v[g][1]) + (v[g][2] + v[g][3]);
      s = wave_sum(s);
      if (WS) {
        if (lane == 0) red[0][rl][half] = s;
        __syncthreads();
        s = red[0][rl][0] + red[0][rl][WPR - 1];
      }
      mean = s / (float)cols;
    }
    float ss = 0.f;
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[g][j] -= mean;
        ss += v[g][j] * v[g][j];
      }
    ss = wave_sum(ss);
    if (WS) {
      if (lane == 0) red[1][rl][half] = ss;
      __syncthreads();
      ss = red[1][rl][0] + red[1][rl][WPR - 1];
    }
    r = rsqrtf(ss / (float)cols + a.eps);
  }
  const half4v_t h = fwht_h16_fragment();
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const int gg = part * GBLK + gb0 + g;  // group of the row
    if (NORM) {
      // modulation of each element: y = ((v * r) * w) * (1 + scale) + shift, the reference's
      // order (kernels.js:82-117)
      const float4 s1 = mods[0][gg * 64 + lane], sh = mods[1][gg * 64 + lane];
      if (a.w) {
        const float4 ww = mods[NV - 1][gg * 64 + lane];
        v[g][0] = v[g][0] * r * ww.x * s1.x + sh.x, v[g][1] = v[g][1] * r * ww.y * s1.y + sh.y;
        v[g][2] = v[g][2] * r * ww.z * s1.z + sh.z, v[g][3] = v[g][3] * r * ww.w * s1.w + sh.w;
      } else {
        v[g][0] = v[g][0] * r * s1.x + sh.x, v[g][1] = v[g][1] * r * s1.y + sh.y;
        v[g][2] = v[g][2] * r * s1.z + sh.z, v[g][3] = v[g][3] * r * s1.w + sh.w;
      }
    }
    if (ROT) fwht256_mfma(v[g], h);
    if (!a.tiled) {
      if (active) store4_f16(a.y, row, gg * 256 + lo, a.ldy, cols, a.tiled, v[g]);
    } else {
      uint2 o;
      o.x = pack_half2(v[g][0], v[g][1]);
      o.y = pack_half2(v[g][2], v[g][3]);
      *reinterpret_cast<uint2*>(&tout[rl * TROW + (gb0 + g) * 256 + lo]) = o;
    }
  }
  if (a.tiled) {
    // write-out of the block's 8 rows: 16-byte unit u = (chunk u / 8, row u % 8), so the 8 units
    // of a chunk are one 128-byte line of the tiled layout and a wave writes 8 whole lines
    __syncthreads();
    const int row0 = (blockIdx.x / PARTS) * 8, c0 = part * GBLK * 32;
    for (int u = threadIdx.x; u < GBLK * 32 * 8; u += rot_threads<G, NORM>()) {
      const int c = u / 8, r = u % 8;
      if (row0 + r >= a.rows) continue;
      const uint4 q = *reinterpret_cast<const uint4*>(&tout[r * TROW + 8 * c]);
      *reinterpret_cast<uint4*>(a.y + tiled_off(row0 + r, 8 * (c0 + c), cols)) = q;
    }
  }
}

template <bool NORM, bool ROT = true>
void launch_rot_rows(const RotRowsArgs& a, int groups) {
  const int parts = (!NORM && groups >= 6 && groups % 2 == 0) ? 2 : 1;  // the kernel's column parts
  const dim3 grid((a.rows + 7) / 8 * parts);
  hipStream_t s = ns2::stream();
  switch (groups) {
#define NS2_ROT_CASE(G) \
    case G: rot_rows_kernel<G, NORM, ROT><<<grid, rot_threads<G, NORM>(), 0, s>>>(a); break;
    NS2_ROT_CASE(1) NS2_ROT_CASE(2) NS2_ROT_CASE(3) NS2_ROT_CASE(4) NS2_ROT_CASE(5) NS2_ROT_CASE(6)
    NS2_ROT_CASE(7) NS2_ROT_CASE(8) NS2_ROT_CASE(9) NS2_ROT_CASE(10) NS2_ROT_CASE(11) NS2_ROT_CASE(12)
    NS2_ROT_CASE(13) NS2_ROT_CASE(14) NS2_ROT_CASE(15) NS2_ROT_CASE(16)
#undef NS2_ROT_CASE
    // rotation only, rows up to 6144 columns (the widest block-linear input)
    case 20: if constexpr (!NORM && ROT) rot_rows_kernel<20, NORM><<<grid, 512, 0, s>>>(a); break;
    case 24: if constexpr (!NORM && ROT) rot_rows_kernel<24, NORM><<<grid, 512, 0, s>>>(a); break;
    default: break;
  }
}

// ---- fp16 operands of the plain linears ------------------------------------------------------

// y = x (- sub) as the tiled fp16 operand [ceil(rows/64)][cols/64][8][64][8] of a tiled linear;
// rows past the last one, up to the 64-row padding, are written as zeros. One block per 64x64
// tile: each wave reads 16 rows of 64 columns (256 contiguous bytes per row, 16 bytes per lane),
// the block transposes the fp16 values through LDS into the tile's chunk-major image and writes
// it out as 8 KB of contiguous 16-byte stores.
__global__ __launch_bounds__(256) void to_tiled_f16_kernel(const float* __restrict__ x, int ldx,
                                                            const float* __restrict__ sub, int lds,
                                                            uint16_t* __restrict__ y, int rows, int cols) {
  constexpr int CS = 64 * 8 + 8;  // halfs per chunk in LDS (16 bytes of padding: the 8 chunks of a
                                 // row fall in different banks)
  __shared__ __attribute__((aligned(16))) uint16_t t[8 * CS];
  const int kb = blockIdx.x % (cols / 64), mb = blockIdx.x / (cols / 64);
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + 256 * i;        // 4-column piece q of the 64x64 tile
    const int r = q / 16, c4 = q % 16;  // row, first column / 4
    const int m = mb * 64 + r;
    uint2 o = make_uint2(0u, 0u);
    if (m < rows) {
      float4 v = *reinterpret_cast<const float4*>(x + (long long)m * ldx + kb * 64 + 4 * c4);
      if (sub) {
        const float4 b = *reinterpret_cast<const float4*>(sub + (long long)m * lds + kb * 64 + 4 * c4);
        v.x -= b.x, v.y -= b.y, v.z -= b.z, v.w -= b.w;
      }
      o = make_uint2(pack_half2(v.x, v.y), pack_half2(v.z, v.w));
    }
    // chunk-major image: chunk c = column / 8 holds 64 rows of 8 halfs
    *reinterpret_cast<uint2*>(&t[(c4 >> 1) * CS + r * 8 + 4 * (c4 & 1)]) = o;
  }
  __syncthreads();
  uint4* dst = reinterpret_cast<uint4*>(y + ((long long)mb * (cols / 64) + kb) * 4096);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int j = tid + 256 * i;  // 16-byte unit: chunk j / 64, row j % 64
    dst[j] = *reinterpret_cast<const uint4*>(&t[(j >> 6) * CS + (j & 63) * 8]);
  }
}

// ---- headNorm -------------------------------------------------------------------------------

// In-place per-head RMSNorm (+ split-half RoPE), kernels.js:307-342. One wave per (row, head).
// Heads h < H1 use w, heads h >= H1 use w2 (two adjacent head ranges with their own weights).
__global__ __launch_bounds__(256) void head_norm_kernel(float* __restrict__ X,
                                                         const float* __restrict__ w1, int H1,
                                                         const float* __restrict__ w2, int L,
                                                         int H, int D, int ld, long long colOff,
                                                         long long rowOff,
                                                         const float* __restrict__ cs,
                                                         long long sinOff, float eps) {
  long long id = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (id >= (long long)L * H) return;
  const int lane = threadIdx.x & 63;
  const int l = (int)(id / H), h = (int)(id % H);
  const float* __restrict__ w = h < H1 ? w1 : w2;
  float* row = X + (rowOff + l) * (long long)ld + colOff + (long long)h * D;
  float ss = 0.f;
  for (int i = lane; i < D; i += 64) ss += row[i] * row[i];
  const float r = rsqrtf(wave_sum(ss) / (float)D + eps);
  if (cs) {
    const int half = D / 2;
    for (int i = lane; i < half; i += 64) {
      const float y1 = row[i] * r * w[i];
      const float y2 = row[i + half] * r * w[i + half];
      const float c = cs[(long long)l * half + i];
      const float s = cs[sinOff + (long long)l * half + i];
      row[i] = y1 * c - y2 * s;
      row[i + half] = y2 * c + y1 * s;
    }
  } else {
    for (int i = lane; i < D; i += 64) row[i] = row[i] * r * w[i];
  }
}

// ---- GLU ----------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void glu_kernel(const float* __restrict__ x,
                                                   float* __restrict__ y, long long n, int I,
                                                   int act) {
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const long long r = i / I, j = i % I;
  const long long base = r * 2 * I + j;
  y[i] = apply_act(x[base], act) * x[base + I];
}

// GLU + rotation + fp16: one wave per 256 output columns.
__global__ __launch_bounds__(256) void glu_rot_kernel(const float* __restrict__ x,
                                                       uint16_t* __restrict__ y, int rows,
                                                       int I, int act, int tiled) {
  const int gpr = I / 256;
  long long g = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= (long long)rows * gpr) return;
  const int lane = threadIdx.x & 63;
  const long long r = g / gpr;
  const int c = (int)(g % gpr) * 256 + lane * 4;
  const float4 a = *reinterpret_cast<const float4*>(x + r * 2 * I + c);
  const float4 b = *reinterpret_cast<const float4*>(x + r * 2 * I + I + c);
  float v[4] = {apply_act(a.x, act) * b.x, apply_act(a.y, act) * b.y,
                apply_act(a.z, act) * b.z, apply_act(a.w, act) * b.w};
  fwht256_wave(v);
  store4_f16(y, r, c, I, I, tiled, v);
}

// ---- elementwise / accumulate / rowSum / RMSNorm ---------------------------------------------

__global__ __launch_bounds__(256) void elementwise_kernel(int op, const float* __restrict__ a,
                                                           const float* __restrict__ b,
                                                           float* __restrict__ y, long long n) {
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float v = a[i];
  if (op == NS2_EW_ADD) v = v + b[i];
  else if (op == NS2_EW_SUB) v = v - b[i];
  else if (op == NS2_EW_SILU) v = silu(v);
  y[i] = v;
}

// The same per element, four elements per thread (16-byte aligned buffers, n % 4 == 0).
__device__ __forceinline__ float ew_op(int op, float v, float w) {
  if (op == NS2_EW_ADD) return v + w;
  if (op == NS2_EW_SUB) return v - w;
  if (op == NS2_EW_SILU) return silu(v);
  return v;
}
__global__ __launch_bounds__(256) void elementwise4_kernel(int op, const float4* __restrict__ a,
                                                            const float4* __restrict__ b,
                                                            float4* __restrict__ y, long long n4) {
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const float4 v = a[i];
  const float4 w = (op == NS2_EW_ADD || op == NS2_EW_SUB) ? b[i] : v;
  y[i] = make_float4(ew_op(op, v.x, w.x), ew_op(op, v.y, w.y), ew_op(op, v.z, w.z), ew_op(op, v.w, w.w));
}

__global__ __launch_bounds__(256) void accumulate_kernel(float* __restrict__ y,
                                                          const float* __restrict__ a,
                                                          long long n) {
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] += a[i];
}

// Y[n] = scale * sum_r w[r] X[r][n]: one thread per column, rows in order (kernels.js:362-376).
// y[n] = scale * sum_r w[r] x[r, n]: one block of 16 waves per 64 columns; wave i sums rows i,
// i + 16, ... of its column, and the 16 partial sums are added in a fixed order.
__global__ __launch_bounds__(1024) void row_sum_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ w,
                                                        float* __restrict__ y, int rows, int N,
                                                        float scale) {
  __shared__ float part[16][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (n < N)
    for (int r = wv; r < rows; r += 16) s += w[r] * x[(long long)r * N + n];
  part[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && n < N) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += part[i][lane];
    y[n] = t * scale;
  }
}

// y[r, i] = a[i] + b[r, i]
__global__ __launch_bounds__(256) void add_rows_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                        float* __restrict__ y, long long total, int n) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < total) y[i] = a[i % n] + b[i];
}

// y[c][r] = x[r][c] for an fp32 [rows, cols] matrix: 64x64 tiles through LDS (one padding
// column against bank conflicts), 256 threads, coalesced reads and writes.
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                        int rows, int cols) {
  __shared__ float tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    // clamped, unconditional loads; the clamped copies land in tile cells that are not stored
    const int r = r0 + ty + 4 * k, c = c0 + tx;
    tile[ty + 4 * k][tx] = x[(long long)(r < rows ? r : rows - 1) * cols + (c < cols ? c : cols - 1)];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int c = c0 + ty + 4 * k, r = r0 + tx;
    if (c < cols && r < rows) y[(long long)c * rows + r] = tile[tx][ty + 4 * k];
  }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       float* __restrict__ y, int cols,
                                                       float eps) {
  __shared__ float red[16];
  const long long base = (long long)blockIdx.x * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) ss += x[base + c] * x[base + c];
  const float r = rsqrtf(block_sum(ss, red) / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += 256) y[base + c] = x[base + c] * r * w[c];
}

// x += rmsnorm(a) * w_add, then y = rmsnorm(x) * w_out (when y is given): the sandwich norms
// around each Gemma3 sublayer (app/models/gemma3.js:76-77, 87-88 and the next layer's input norm).
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(float* __restrict__ x,
                                                          const float* __restrict__ a,
                                                          const float* __restrict__ w_add,
                                                          const float* __restrict__ w_out,
                                                          float* __restrict__ y, int cols, float eps) {
  __shared__ float red[16];
  const long long base = (long long)blockIdx.x * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) ss += a[base + c] * a[base + c];
  const float r = rsqrtf(block_sum(ss, red) / (float)cols + eps);
  float sx = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float v = x[base + c] + a[base + c] * r * w_add[c];
    x[base + c] = v;
    sx += v * v;
  }
  if (!y) return;
  const float rx = rsqrtf(block_sum(sx, red) / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += 256) y[base + c] = x[base + c] * rx * w_out[c];
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7) == 0; }

inline unsigned blocks_for(long long n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

extern "C" {

int ns2_hadamard256(const float* x, float* y, long long groups) {
  NS2_READY();
  if (groups <= 0) return NS2_OK;
  NS2_REQUIRE(x && y && aligned16(x) && aligned16(y), "ns2_hadamard256: null or unaligned buffer");
  ns2::ProfScope prof_("hadamard256");
  hadamard256_kernel<<<blocks_for(groups, 4), 256, 0, ns2::stream()>>>(x, y, groups);
  NS2_LAUNCHED("hadamard256");
  return NS2_OK;
}

int ns2_rotate_f16(const float* x, int ldx, uint16_t* y, int ldy, int rows, int cols, int tiled) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(cols > 0 && cols % 256 == 0, "ns2_rotate_f16: cols=%d must be a multiple of 256", cols);
  NS2_REQUIRE(ldx % 4 == 0 && ldx >= cols && (tiled || (ldy % 4 == 0 && ldy >= cols)),
              "ns2_rotate_f16: ldx=%d ldy=%d must be multiples of 4 and >= cols", ldx, ldy);
  NS2_REQUIRE(x && y && aligned16(x) && aligned8(y), "ns2_rotate_f16: null or unaligned buffer");
  const int gpr = cols / 256;
  ns2::ProfScope prof_("rotate_f16");
  if (gpr <= 16 || gpr == 20 || gpr == 24) {
    RotRowsArgs a{x, ldx, nullptr, 0, 0, nullptr, 0.f, y, ldy, rows, tiled};
    launch_rot_rows<false>(a, gpr);
  } else {
    rotate_f16_kernel<<<blocks_for((long long)rows * gpr, 4), 256, 0, ns2::stream()>>>(x, ldx, y, ldy, rows, gpr, tiled);
  }
  NS2_LAUNCHED("rotate_f16");
  return NS2_OK;
}

int ns2_norm_mod(const float* x, const float* mod, long long shiftOff, long long scaleOff,
                 int rows, int cols, const float* weight, float eps, float* y) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(x && mod && y && cols > 0, "ns2_norm_mod: bad arguments");
  ns2::ProfScope prof_("norm_mod");
  const bool rows_ok = cols % 256 == 0 && cols <= 256 * 8 && aligned16(x) && aligned16(mod) && aligned16(y) &&
                       shiftOff % 4 == 0 && scaleOff % 4 == 0 && (!weight || aligned16(weight));
  const dim3 grid((rows + 7) / 8), block(512);
  hipStream_t s = ns2::stream();
  switch (rows_ok ? cols / 256 : 0) {
#define NS2_NM_CASE(G) \
    case G: norm_mod_rows_kernel<G><<<grid, block, 0, s>>>(x, mod, shiftOff, scaleOff, rows, weight, eps, y); break;
    NS2_NM_CASE(1) NS2_NM_CASE(2) NS2_NM_CASE(3) NS2_NM_CASE(4) NS2_NM_CASE(5) NS2_NM_CASE(6) NS2_NM_CASE(7)
    NS2_NM_CASE(8)
#undef NS2_NM_CASE
    default: norm_mod_kernel<<<rows, 256, 0, s>>>(x, mod, shiftOff, scaleOff, cols, weight, eps, y);
  }
  NS2_LAUNCHED("norm_mod");
  return NS2_OK;
}

int ns2_norm_mod_rotate_f16(const float* x, const float* mod, long long shiftOff,
                            long long scaleOff, int rows, int cols, const float* weight,
                            float eps, uint16_t* y, int tiled) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(cols % 256 == 0 && cols >= 256 && cols <= 4096,
              "ns2_norm_mod_rotate_f16: cols=%d must be a multiple of 256 in [256, 4096]", cols);
  NS2_REQUIRE(x && mod && y && aligned16(x) && aligned8(y) && shiftOff % 4 == 0 && scaleOff % 4 == 0 &&
                  aligned16(mod) && (!weight || aligned16(weight)),
              "ns2_norm_mod_rotate_f16: null or unaligned buffer/offset");
  ns2::ProfScope prof_("norm_mod_rotate_f16");
  RotRowsArgs a{x, cols, mod, shiftOff, scaleOff, weight, eps, y, cols, rows, tiled};
  launch_rot_rows<true>(a, cols / 256);
  NS2_LAUNCHED("norm_mod_rotate_f16");
  return NS2_OK;
}

int ns2_norm_mod_f16(const float* x, const float* mod, long long shiftOff, long long scaleOff, int rows, int cols,
                     const float* weight, float eps, uint16_t* y, int tiled) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(cols % 256 == 0 && cols >= 256 && cols <= 4096,
              "ns2_norm_mod_f16: cols=%d must be a multiple of 256 in [256, 4096]", cols);
  NS2_REQUIRE(x && mod && y && aligned16(x) && aligned8(y) && shiftOff % 4 == 0 && scaleOff % 4 == 0 &&
                  aligned16(mod) && (!weight || aligned16(weight)),
              "ns2_norm_mod_f16: null or unaligned buffer/offset");
  ns2::ProfScope prof_("norm_mod_f16");
  RotRowsArgs a{x, cols, mod, shiftOff, scaleOff, weight, eps, y, cols, rows, tiled};
  launch_rot_rows<true, false>(a, cols / 256);
  NS2_LAUNCHED("norm_mod_f16");
  return NS2_OK;
}

int ns2_to_tiled_f16(const float* x, int ldx, const float* sub, int ldsub, uint16_t* y, int rows, int cols) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(cols > 0 && cols % 64 == 0, "ns2_to_tiled_f16: cols=%d must be a multiple of 64", cols);
  NS2_REQUIRE(ldx >= cols && ldx % 4 == 0 && (!sub || (ldsub >= cols && ldsub % 4 == 0)),
              "ns2_to_tiled_f16: ldx=%d / ldsub=%d must be multiples of 4 and >= cols", ldx, ldsub);
  NS2_REQUIRE(x && y && aligned16(x) && aligned16(y) && (!sub || aligned16(sub)),
              "ns2_to_tiled_f16: null or unaligned buffer");
  const long long tiles = (long long)(rows + 63) / 64 * (cols / 64);
  ns2::ProfScope prof_("to_tiled_f16");
  to_tiled_f16_kernel<<<(unsigned)tiles, 256, 0, ns2::stream()>>>(x, ldx, sub, ldsub, y, rows, cols);
  NS2_LAUNCHED("to_tiled_f16");
  return NS2_OK;
}

int ns2_head_norm(float* X, const float* w, int L, int H, int D, int ld, long long colOff,
                  long long rowOff, const float* cs, long long sinOff, float eps) {
  NS2_READY();
  if (L <= 0 || H <= 0) return NS2_OK;
  NS2_REQUIRE(X && w && D > 0 && D % 2 == 0, "ns2_head_norm: bad arguments");
  ns2::ProfScope prof_("head_norm");
  head_norm_kernel<<<blocks_for((long long)L * H, 4), 256, 0, ns2::stream()>>>(X, w, H, w, L, H, D, ld, colOff, rowOff, cs, sinOff, eps);
  NS2_LAUNCHED("head_norm");
  return NS2_OK;
}

int ns2_head_norm2(float* X, const float* w1, int H1, const float* w2, int H2, int L, int D, int ld,
                   long long colOff, long long rowOff, const float* cs, long long sinOff, float eps) {
  NS2_READY();
  if (L <= 0 || H1 + H2 <= 0) return NS2_OK;
  NS2_REQUIRE(X && (H1 <= 0 || w1) && (H2 <= 0 || w2) && H1 >= 0 && H2 >= 0 && D > 0 && D % 2 == 0,
              "ns2_head_norm2: bad arguments");
  const int H = H1 + H2;
  ns2::ProfScope prof_("head_norm");
  head_norm_kernel<<<blocks_for((long long)L * H, 4), 256, 0, ns2::stream()>>>(X, w1, H1, w2, L, H, D, ld, colOff, rowOff, cs, sinOff, eps);
  NS2_LAUNCHED("head_norm2");
  return NS2_OK;
}

int ns2_glu(const float* x, float* y, int rows, int I, int act) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(x && y && I > 0, "ns2_glu: bad arguments");
  const long long n = (long long)rows * I;
  ns2::ProfScope prof_("glu");
  glu_kernel<<<blocks_for(n, 256), 256, 0, ns2::stream()>>>(x, y, n, I, act);
  NS2_LAUNCHED("glu");
  return NS2_OK;
}

int ns2_glu_rotate_f16(const float* x, uint16_t* y, int rows, int I, int act, int tiled) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(I > 0 && I % 256 == 0, "ns2_glu_rotate_f16: I=%d must be a multiple of 256", I);
  NS2_REQUIRE(x && y && aligned16(x) && aligned8(y), "ns2_glu_rotate_f16: null or unaligned buffer");
  const long long groups = (long long)rows * (I / 256);
  ns2::ProfScope prof_("glu_rotate_f16");
  glu_rot_kernel<<<blocks_for(groups, 4), 256, 0, ns2::stream()>>>(x, y, rows, I, act, tiled);
  NS2_LAUNCHED("glu_rotate_f16");
  return NS2_OK;
}

int ns2_elementwise(int op, const float* a, const float* b, float* y, long long n) {
  NS2_READY();
  if (n <= 0) return NS2_OK;
  NS2_REQUIRE(op >= NS2_EW_ADD && op <= NS2_EW_COPY, "ns2_elementwise: unknown op %d", op);
  NS2_REQUIRE(a && y && (b || op == NS2_EW_SILU || op == NS2_EW_COPY), "ns2_elementwise: null buffer");
  ns2::ProfScope prof_("elementwise");
  if (n % 4 == 0 && aligned16(a) && aligned16(y) && (!b || aligned16(b))) {
    elementwise4_kernel<<<blocks_for(n / 4, 256), 256, 0, ns2::stream()>>>(
        op, reinterpret_cast<const float4*>(a), reinterpret_cast<const float4*>(b), reinterpret_cast<float4*>(y), n / 4);
  } else {
    elementwise_kernel<<<blocks_for(n, 256), 256, 0, ns2::stream()>>>(op, a, b, y, n);
  }
  NS2_LAUNCHED("elementwise");
  return NS2_OK;
}

int ns2_accumulate(float* y, const float* a, long long n) {
  NS2_READY();
  if (n <= 0) return NS2_OK;
  NS2_REQUIRE(a && y, "ns2_accumulate: null buffer");
  ns2::ProfScope prof_("accumulate");
  accumulate_kernel<<<blocks_for(n, 256), 256, 0, ns2::stream()>>>(y, a, n);
  NS2_LAUNCHED("accumulate");
  return NS2_OK;
}

int ns2_add_rows(const float* a, const float* b, float* y, int rows, int n) {
  NS2_READY();
  if (rows <= 0 || n <= 0) return NS2_OK;
  NS2_REQUIRE(a && b && y, "ns2_add_rows: null buffer");
  const long long total = (long long)rows * n;
  ns2::ProfScope prof_("add_rows");
  add_rows_kernel<<<blocks_for(total, 256), 256, 0, ns2::stream()>>>(a, b, y, total, n);
  NS2_LAUNCHED("add_rows");
  return NS2_OK;
}

int ns2_transpose(const float* x, float* y, int rows, int cols) {
  NS2_READY();
  if (rows <= 0 || cols <= 0) return NS2_OK;
  NS2_REQUIRE(x && y && x != y, "ns2_transpose: null or aliased buffers");
  ns2::ProfScope prof_("transpose");
  transpose_kernel<<<dim3((cols + 63) / 64, (rows + 63) / 64), 256, 0, ns2::stream()>>>(x, y, rows, cols);
  NS2_LAUNCHED("transpose");
  return NS2_OK;
}

int ns2_row_sum(const float* x, const float* w, float* y, int rows, int N, float scale) {
  NS2_READY();
  if (N <= 0) return NS2_OK;
  NS2_REQUIRE(x && w && y && rows >= 0, "ns2_row_sum: bad arguments");
  ns2::ProfScope prof_("row_sum");
  row_sum_kernel<<<blocks_for(N, 64), 1024, 0, ns2::stream()>>>(x, w, y, rows, N, scale);
  NS2_LAUNCHED("row_sum");
  return NS2_OK;
}

int ns2_rmsnorm(const float* x, const float* w, float* y, int rows, int cols, float eps) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(x && w && y && cols > 0, "ns2_rmsnorm: bad arguments");
  ns2::ProfScope prof_("rmsnorm");
  rmsnorm_kernel<<<rows, 256, 0, ns2::stream()>>>(x, w, y, cols, eps);
  NS2_LAUNCHED("rmsnorm");
  return NS2_OK;
}

int ns2_add_rmsnorm(float* x, const float* a, const float* w_add, const float* w_out, float* y, int rows,
                    int cols, float eps) {
  NS2_READY();
  if (rows <= 0) return NS2_OK;
  NS2_REQUIRE(x && a && w_add && cols > 0 && (!y || w_out), "ns2_add_rmsnorm: bad arguments");
  NS2_REQUIRE(y != x && y != a && a != x, "ns2_add_rmsnorm: x, a and y must not alias");
  ns2::ProfScope prof_("add_rmsnorm");
  add_rmsnorm_kernel<<<rows, 256, 0, ns2::stream()>>>(x, a, w_add, w_out, y, cols, eps);
  NS2_LAUNCHED("add_rmsnorm");
  return NS2_OK;
}

}  // extern "C"
