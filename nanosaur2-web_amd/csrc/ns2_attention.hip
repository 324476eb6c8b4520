// Joint image+text flash attention on MFMA (fp16 operands, fp32 accumulation).
//
// Two kernels per call:
//  1. pack: reads the fp32 q/k/v views, applies the optional per-head RMSNorm and split-half
//     RoPE (the DiT's headNorm, kernels.js:307-342), folds scale*log2(e) into q, and writes
//     fp16 operands. Q is row-major per head, Qp [B*H][Lq_pad][D]. K and V are written per
//     64-key tile as the exact byte image of the flash kernel's LDS stage, so a tile moves
//     into LDS with direct global->LDS loads (no registers, no LDS store instructions):
//        Kc [B*H][tile][D/8 chunks][64 keys][8 dims]        (chunk-major K)
//        Vc [B*H][tile][8 key-chunks][D dims][8 keys]       (V transposed, chunk-major)
//     plus one fp32 bias per key in log2 units (0 on image keys, the log-prompt-weight on
//     text keys, -1e30 on padding keys).
//  2. flash: one workgroup per (query block, head, batch). Each wave owns QT x 32 queries and
//     works in the transposed domain, so no register shuffles are needed between products:
//        S^T = K Q^T       (A = K fragments from LDS, B = Q^T held in registers)
//        O^T += V^T P^T    (A = V^T fragments from LDS, B = P^T straight from S^T registers)
//     The 32x32 MFMA accumulator of S^T gives every lane one query column and 16 keys, which
//     is exactly the k-slice a lane supplies as B operand of the next product (the k order
//     inside an MFMA is free as long as A and B agree), and the online-softmax statistics
//     of a query live in the same lanes as its output column. In the chunk-major LDS images
//     the 32 lanes of a half-wave read 32 consecutive 16-byte rows: no bank conflicts.
#include <stdlib.h>

#include <type_traits>

#include "ns2_common.h"

using namespace ns2dev;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaskBias = -1.0e30f;
constexpr int KB = 64;          // keys per tile
constexpr int QPAD = 256;       // Lq padding granule (largest query block)

// Position of key k (within a 16-key step) in the stored V^T order: bits 2 and 3 swapped, so
// the 8 keys one lane feeds to a PV product, {4hi..4hi+3, 8+4hi..8+4hi+3}, are 8 adjacent
// stored keys (one 16-byte chunk). The map is its own inverse.
__device__ __forceinline__ int vkey_pos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

struct PackArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* key_bias;
  const float* q_norm;
  const float* k_norm;
  const float* cs;
  half_t* Qp;
  half_t* Kc;
  half_t* Vc;
  float* bias2;
  long long qOff, kOff, vOff, qBatch, kBatch, vBatch, biasBatch, sinOff;
  int Lq, Lk, Lq_pad, Lk_pad, H, ldq, ldk, ldv, biasStart, rope_rows;
  float qscale, eps;
  int skip_q;  // the flash kernel prepares Q itself (vectorized pack only)
  // K and V rows from kv2_start on come from a second view (the DiT's text keys, projected
  // apart from the image rows): row r at k2 / v2 + (r - kv2_start) * ld2; null: one view
  const float* k2;
  const float* v2;
  int ld2, kv2_start;
  // values of keys [0, v_pre) are already in Vc (written by the producing GEMM); v_pre % 16 == 0
  // (vectorized pack only)
  int v_pre;
};

// Row r of head 0 in the K and V views of batch element b.
__device__ __forceinline__ const float* key_row(const PackArgs& a, int b, int r) {
  return a.k2 && r >= a.kv2_start ? a.k2 + (long long)(r - a.kv2_start) * a.ld2
                                  : a.k + a.kOff + b * a.kBatch + (long long)r * a.ldk;
}
__device__ __forceinline__ const float* value_row(const PackArgs& a, int b, int r) {
  return a.v2 && r >= a.kv2_start ? a.v2 + (long long)(r - a.kv2_start) * a.ld2
                                  : a.v + a.vOff + b * a.vBatch + (long long)r * a.ldv;
}

// Per-row prologue for one head row of D values, 4 threads per row: thread part p owns
// the rope pairs i in [p*D/8, (p+1)*D/8), i.e. dims i and i + D/2.
template <int D>
__device__ __forceinline__ void prep_row(const float* __restrict__ src, const float* __restrict__ nw,
                                         const float* __restrict__ cs, long long sinOff, int row,
                                         bool rope, float mul, float eps, int part,
                                         half_t* __restrict__ dst) {
  constexpr int HALF = D / 2, PER = D / 8;
  float x1[PER], x2[PER];
  const int i0 = part * PER;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    x1[j] = src[i0 + j];
    x2[j] = src[HALF + i0 + j];
  }
  if (nw) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss += x1[j] * x1[j] + x2[j] * x2[j];
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    const float r = rsqrtf(ss / (float)D + eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      x1[j] = x1[j] * r * nw[i0 + j];
      x2[j] = x2[j] * r * nw[HALF + i0 + j];
    }
  }
  if (rope) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const float c = cs[(long long)row * HALF + i0 + j];
      const float s = cs[sinOff + (long long)row * HALF + i0 + j];
      const float y1 = x1[j] * c - x2[j] * s;
      const float y2 = x2[j] * c + x1[j] * s;
      x1[j] = y1;
      x2[j] = y2;
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    dst[i0 + j] = (half_t)(x1[j] * mul);
    dst[HALF + i0 + j] = (half_t)(x2[j] * mul);
  }
}

// grid: (rows / 64, H, batch), 256 threads: 64 rows x 4 parts. Block x handles key tile x.
template <int D>
__global__ __launch_bounds__(256) void attn_pack_kernel(PackArgs a) {
  constexpr int KROW = D + 8;
  __shared__ __attribute__((aligned(16))) half_t ktile[KB][KROW];
  __shared__ half_t vs[D][KB + 2];
  const int h = blockIdx.y, b = blockIdx.z;
  const int bh = b * a.H + h;
  const int tile = blockIdx.x, row0 = tile * KB;
  const int tid = threadIdx.x;
  const int rl = tid >> 2, part = tid & 3;
  const int row = row0 + rl;

  // Q rows (row-major per head)
  if (row0 < a.Lq_pad) {
    half_t* dst = a.Qp + ((long long)bh * a.Lq_pad + row) * D;
    if (row < a.Lq) {
      const float* src = a.q + a.qOff + b * a.qBatch + (long long)row * a.ldq + (long long)h * D;
      prep_row<D>(src, a.q_norm, a.cs, a.sinOff, row, a.cs && row < a.rope_rows, a.qscale, a.eps, part, dst);
    } else {
#pragma unroll
      for (int j = 0; j < D / 4; ++j) dst[part * (D / 4) + j] = (half_t)0.f;
    }
  }
  if (row0 >= a.Lk_pad) return;  // uniform per block

  // K rows -> LDS, V rows -> LDS transposed
  if (row < a.Lk) {
    const float* src = key_row(a, b, row) + (long long)h * D;
    prep_row<D>(src, a.k_norm, a.cs, a.sinOff, row, a.cs && row < a.rope_rows, 1.0f, a.eps, part, &ktile[rl][0]);
  } else {
#pragma unroll
    for (int j = 0; j < D / 4; ++j) ktile[rl][part * (D / 4) + j] = (half_t)0.f;
  }
  {
    const float* src = value_row(a, b, row < a.Lk ? row : a.Lk - 1) + (long long)h * D;
#pragma unroll
    for (int j = 0; j < D / 4; ++j) {
      const int d = part * (D / 4) + j;
      vs[d][rl] = (half_t)(row < a.Lk ? src[d] : 0.f);
    }
  }
  __syncthreads();

  // chunk-major tile images, 16 bytes per thread and step
  const long long tiles = a.Lk_pad / KB;
  half_t* kdst = a.Kc + ((long long)bh * tiles + tile) * (KB * D);
  for (int i = tid; i < (D / 8) * KB; i += 256) {
    const int key = i % KB, chunk = i / KB;
    *reinterpret_cast<uint4*>(kdst + (long long)i * 8) = *reinterpret_cast<const uint4*>(&ktile[key][chunk * 8]);
  }
  half_t* vdst = a.Vc + ((long long)bh * tiles + tile) * (KB * D);
  for (int i = tid; i < 8 * D; i += 256) {
    const int d = i % D, kc = i / D;
    half8_t v8;
#pragma unroll
    for (int e = 0; e < 8; ++e) v8[e] = vs[d][vkey_pos(kc * 8 + e)];
    *reinterpret_cast<half8_t*>(vdst + (long long)i * 8) = v8;
  }
  // per-key bias in log2 units (one head does it)
  if (h == 0 && tid < KB) {
    const int key = row0 + tid;
    float bv = kMaskBias;
    if (key < a.Lk) {
      bv = 0.f;
      if (a.key_bias && key >= a.biasStart) bv = a.key_bias[b * a.biasBatch + key - a.biasStart] * kLog2e;
    }
    a.bias2[(long long)b * a.Lk_pad + key] = bv;
  }
}

// One key row's share for four lanes (adjacent, within a quad): lane part q owns rope pairs
// [q D/8, (q+1) D/8), i.e. dims q D/8 .. +D/8 of each half. Every load is issued first (the
// row, the norm weights, the rope table): none depends on another, so their latencies overlap
// instead of following the row's reduction.
template <int D>
__device__ __forceinline__ void prep_quarter_row(const float* __restrict__ src, const float* __restrict__ nw,
                                                 const float* __restrict__ cs, long long sinOff, int row,
                                                 bool rope, float eps, int q, float* x1, float* x2) {
  constexpr int HALF = D / 2, PER = D / 8;
  const int i0 = q * PER;
  float w1[PER], w2[PER], c[PER], sn[PER];
#pragma unroll
  for (int j = 0; j < PER; j += 4) {
    const float4 a = *reinterpret_cast<const float4*>(src + i0 + j);
    const float4 b = *reinterpret_cast<const float4*>(src + HALF + i0 + j);
    x1[j] = a.x, x1[j + 1] = a.y, x1[j + 2] = a.z, x1[j + 3] = a.w;
    x2[j] = b.x, x2[j + 1] = b.y, x2[j + 2] = b.z, x2[j + 3] = b.w;
  }
  if (nw) {
#pragma unroll
    for (int j = 0; j < PER; j += 4) {
      const float4 a = *reinterpret_cast<const float4*>(nw + i0 + j);
      const float4 b = *reinterpret_cast<const float4*>(nw + HALF + i0 + j);
      w1[j] = a.x, w1[j + 1] = a.y, w1[j + 2] = a.z, w1[j + 3] = a.w;
      w2[j] = b.x, w2[j + 1] = b.y, w2[j + 2] = b.z, w2[j + 3] = b.w;
    }
  }
  if (rope) {
    const float* cp = cs + (long long)row * HALF + i0;
    const float* sp = cs + sinOff + (long long)row * HALF + i0;
#pragma unroll
    for (int j = 0; j < PER; j += 4) {
      const float4 a = *reinterpret_cast<const float4*>(cp + j);
      const float4 b = *reinterpret_cast<const float4*>(sp + j);
      c[j] = a.x, c[j + 1] = a.y, c[j + 2] = a.z, c[j + 3] = a.w;
      sn[j] = b.x, sn[j + 1] = b.y, sn[j + 2] = b.z, sn[j + 3] = b.w;
    }
  }
  if (nw) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss += x1[j] * x1[j] + x2[j] * x2[j];
    ss += dpp<kDppXor1>(ss);  // the row's other three lanes
    ss += dpp<kDppXor2>(ss);
    const float r = rsqrtf(ss / (float)D + eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      x1[j] = x1[j] * r * w1[j];
      x2[j] = x2[j] * r * w2[j];
    }
  }
  if (rope) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const float y1 = x1[j] * c[j] - x2[j] * sn[j];
      const float y2 = x2[j] * c[j] + x1[j] * sn[j];
      x1[j] = y1;
      x2[j] = y2;
    }
  }
}

__device__ __forceinline__ uint4 pack8_f16(const float* x) {
  return make_uint4(pack_half2(x[0], x[1]), pack_half2(x[2], x[3]), pack_half2(x[4], x[5]), pack_half2(x[6], x[7]));
}

// Vectorized pack for 16-byte aligned views (every view of the DiT path): no LDS, no
// barrier, every global access 16 bytes per lane except the V gathers (D/32 floats). One
// block per (64-row tile, head, batch):
//   all waves: K rows, four lanes per row (norm and RoPE applied), stored straight into the
//   chunk-major tile (the flash kernel reads Q itself from these aligned views);
//   all waves: V, lane (kc, dg) gathers the 8 keys of stored key-chunk kc for dims
//   [dg D/32, (dg+1) D/32) and writes them as the 16-byte rows of the transposed tile.
template <int D>
__global__ __launch_bounds__(256) void attn_pack_vec_kernel(PackArgs a) {
  constexpr int HALF = D / 2, DPL = D / 32;
  const int h = blockIdx.y, b = blockIdx.z;
  const int bh = b * a.H + h;
  const int tile = blockIdx.x, row0 = tile * KB;
  const int tid = threadIdx.x;
  const long long tiles = a.Lk_pad / KB;
  const bool kv = row0 < a.Lk_pad;  // uniform per block

  // V gathers first: they do not depend on the Q/K work. Keys past Lk read the last key (the
  // loads stay unconditional and issue back to back) and are zeroed afterwards.
  const int kc = tid >> 5, dg = tid & 31;
  // chunk kc holds keys of the 16-key group row0 + 16 (kc / 2) only
  const bool vput = kv && row0 + 16 * (kc >> 1) >= a.v_pre;
  float vv[8][DPL];
  if (vput) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = row0 + vkey_pos(kc * 8 + e);
      const int kr = key < a.Lk ? key : a.Lk - 1;
      const float* src = value_row(a, b, kr) + (long long)h * D + dg * DPL;
#pragma unroll
      for (int j = 0; j < DPL; ++j) vv[e][j] = src[j];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = row0 + vkey_pos(kc * 8 + e);
#pragma unroll
      for (int j = 0; j < DPL; ++j) vv[e][j] = key < a.Lk ? vv[e][j] : 0.f;
    }
  }

  // K rows, four lanes per row, stored as 4-half pieces of the 8-dim chunks: chunk c (dims
  // 8c..8c+7) of key rl sits at (c * 64 + rl) * 8 in the tile
  if (kv) {
    constexpr int PER = D / 8;
    const int rl = tid >> 2, q = tid & 3;
    const int row = row0 + rl;
    float x1[PER], x2[PER];
    if (row < a.Lk) {
      const float* src = key_row(a, b, row) + (long long)h * D;
      prep_quarter_row<D>(src, a.k_norm, a.cs, a.sinOff, row, a.cs && row < a.rope_rows, a.eps, q, x1, x2);
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) x1[j] = x2[j] = 0.f;
    }
    half_t* kdst = a.Kc + ((long long)bh * tiles + tile) * (KB * D) + rl * 8;
#pragma unroll
    for (int j = 0; j < PER; j += 4) {
      const int d1 = q * PER + j, d2 = HALF + d1;
      *reinterpret_cast<uint2*>(kdst + (d1 / 8) * (KB * 8) + d1 % 8) =
          make_uint2(pack_half2(x1[j], x1[j + 1]), pack_half2(x1[j + 2], x1[j + 3]));
      *reinterpret_cast<uint2*>(kdst + (d2 / 8) * (KB * 8) + d2 % 8) =
          make_uint2(pack_half2(x2[j], x2[j + 1]), pack_half2(x2[j + 2], x2[j + 3]));
    }
  }

  if (vput) {
    half_t* vdst = a.Vc + ((long long)bh * tiles + tile) * (KB * D) + ((long long)kc * D + dg * DPL) * 8;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      float col[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) col[e] = vv[e][j];
      *reinterpret_cast<uint4*>(vdst + j * 8) = pack8_f16(col);
    }
  }
  if (kv) {
    // per-key bias in log2 units (one head does it)
    if (h == 0 && tid < KB) {
      const int key = row0 + tid;
      float bv = kMaskBias;
      if (key < a.Lk) {
        bv = 0.f;
        if (a.key_bias && key >= a.biasStart) bv = a.key_bias[b * a.biasBatch + key - a.biasStart] * kLog2e;
      }
      a.bias2[(long long)b * a.Lk_pad + key] = bv;
    }
  }
}

struct FlashArgs {
  const half_t* Qp;
  const half_t* Kc;
  const half_t* Vc;
  const float* bias2;
  float* O;
  long long oOff, oBatch;
  int Lq, Lk, Lq_pad, Lk_pad, H, ldo;
  int bias_block0;  // first key tile that needs the per-key bias (text or padding keys)
  int qblocks;      // query blocks per (batch, head)
  int pairs;        // batch * heads
  int xcd_order;    // 1: block id -> (pair, query block) keeps a pair on one XCD
  // qraw: Q comes straight from the fp32 view (16-byte aligned) and the kernel applies the
  // optional per-head RMSNorm, RoPE and scale*log2(e) itself; otherwise it reads Qp
  int qraw;
  const float* q;
  const float* q_norm;
  const float* cs;
  long long qOff, qBatch, sinOff;
  int ldq, rope_rows;
  float qscale, eps;
};

// Q^T operands of a wave: lane holds query q0 + qt*32 + lq, dims c*16 + 8*hi .. +7. With qraw
// the lane reads those 8*DC fp32 values and prepares them as the pack does (kernels.js:307-342):
// RMSNorm over the head row (its other half is in lane ^ 32), then split-half RoPE, whose
// partner of dim 16c + 8hi + e is dim 16(c + DC/2) + 8hi + e of the same lane, then the
// scale; rows past Lq are zero.
template <int D, int QT>
__device__ __forceinline__ void load_q(const FlashArgs& a, int b, int h, int bh, int q0, int lq, int hi,
                                       half8_t (&qf)[QT][D / 16]) {
  constexpr int DC = D / 16;
  static_assert(DC % 2 == 0, "RoPE halves must be whole k-steps");
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = q0 + qt * 32 + lq;
    if (a.qraw) {
      float x[DC][8];
      if (q < a.Lq) {
        const float* src = a.q + a.qOff + (long long)b * a.qBatch + (long long)q * a.ldq + (long long)h * D + 8 * hi;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          const float4 u = *reinterpret_cast<const float4*>(src + 16 * c);
          const float4 w = *reinterpret_cast<const float4*>(src + 16 * c + 4);
          x[c][0] = u.x, x[c][1] = u.y, x[c][2] = u.z, x[c][3] = u.w;
          x[c][4] = w.x, x[c][5] = w.y, x[c][6] = w.z, x[c][7] = w.w;
        }
      } else {
#pragma unroll
        for (int c = 0; c < DC; ++c)
#pragma unroll
          for (int e = 0; e < 8; ++e) x[c][e] = 0.f;
      }
      if (a.q_norm) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < DC; ++c)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += x[c][e] * x[c][e];
        ss += __shfl_xor(ss, 32, 64);
        const float r = rsqrtf(ss / (float)D + a.eps);
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          const float4 w1 = *reinterpret_cast<const float4*>(a.q_norm + 16 * c + 8 * hi);
          const float4 w2 = *reinterpret_cast<const float4*>(a.q_norm + 16 * c + 8 * hi + 4);
          const float wv[8] = {w1.x, w1.y, w1.z, w1.w, w2.x, w2.y, w2.z, w2.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) x[c][e] = x[c][e] * r * wv[e];
        }
      }
      if (a.cs && q < a.rope_rows) {
        constexpr int HALF = D / 2;
#pragma unroll
        for (int c = 0; c < DC / 2; ++c) {
          const float* cp = a.cs + (long long)q * HALF + 16 * c + 8 * hi;
          const float* sp = a.cs + a.sinOff + (long long)q * HALF + 16 * c + 8 * hi;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float cv = cp[e], sv = sp[e];
            const float y1 = x[c][e] * cv - x[c + DC / 2][e] * sv;
            const float y2 = x[c + DC / 2][e] * cv + x[c][e] * sv;
            x[c][e] = y1;
            x[c + DC / 2][e] = y2;
          }
        }
      }
#pragma unroll
      for (int c = 0; c < DC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[qt][c][e] = (half_t)(x[c][e] * a.qscale);
    } else {
      const half_t* qrow = a.Qp + ((long long)bh * a.Lq_pad + q) * D + 8 * hi;
#pragma unroll
      for (int c = 0; c < DC; ++c) qf[qt][c] = *reinterpret_cast<const half8_t*>(qrow + c * 16);
    }
  }

}

// Tile t -> LDS stage st with direct global->LDS loads: the stage image is BLOCKS blocks of
// 1 KB (K blocks, then V^T blocks) plus the 256-byte key bias; wave w of NW moves blocks w,
// w+NW, ..., BLOCKS (the bias); lane l moves bytes [16l, 16l+16) of a block (16 lanes for the
// bias). The per-wave sources and destinations are fixed up front; a tile adds its offsets.
template <int D, int NW>
struct TileLoader {
  static constexpr int TILE = KB * D;            // halfs per K (or V) tile image
  static constexpr int BLOCKS = 2 * TILE / 512;  // 1 KB blocks per tile (K then V)
  static constexpr int NJ = (BLOCKS + NW) / NW;  // loads per wave per tile, at most
  const char* g_src[NJ];
  uint32_t l_dst[NJ];
  int g_step[NJ], l_step[NJ];
  int wave, lane;

  __device__ __forceinline__ TileLoader(const half_t* Kt, const half_t* Vt, const float* Bg, uint32_t ks_base,
                                        uint32_t vts_base, uint32_t kb_base, int wave_, int lane_)
      : wave(wave_), lane(lane_) {
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int j = wave + i * NW;
      if (j < BLOCKS / 2) {
        g_src[i] = reinterpret_cast<const char*>(Kt + j * 512);
        l_dst[i] = ks_base + j * 1024;
      } else if (j < BLOCKS) {
        g_src[i] = reinterpret_cast<const char*>(Vt + (j - BLOCKS / 2) * 512);
        l_dst[i] = vts_base + (j - BLOCKS / 2) * 1024;
      } else {
        g_src[i] = reinterpret_cast<const char*>(Bg);
        l_dst[i] = kb_base;
      }
      g_step[i] = j < BLOCKS ? TILE * 2 : KB * 4;  // bytes per tile in global memory
      l_step[i] = j < BLOCKS ? TILE * 2 : KB * 4;  // bytes per LDS stage
    }
  }
  // load i (< NJ) of this wave for tile t into stage st; loads past the wave's share are none
  __device__ __forceinline__ void issue_one(int i, int t, int st) const {
    const int j = wave + i * NW;
    if (j > BLOCKS) return;
    if (j < BLOCKS || lane < KB / 4)
      dma16(g_src[i] + (long long)t * g_step[i] + lane * 16, __builtin_amdgcn_readfirstlane(l_dst[i] + st * l_step[i]));
  }
  __device__ __forceinline__ void issue(int t, int st) const {
#pragma unroll
    for (int i = 0; i < NJ; ++i) issue_one(i, t, st);
  }
  // Wait until at most the loads of the N most recent tiles are in flight for this wave
  // (wave w issues (BLOCKS - w) / NW + 1 loads per tile).
  template <int N>
  __device__ __forceinline__ void wait_newer() const {
    if (wave <= BLOCKS % NW) vm_wait<N * (BLOCKS / NW + 1)>();
    else vm_wait<N * (BLOCKS / NW)>();
  }
};

// Scores are kept relative to a per-query reference m_ref (log2 units) that only moves when a
// score exceeds it by more than 2^kRebase; between moves the output accumulator needs no
// rescale. Any reference gives the same softmax, and p <= 2^kRebase stays in fp16 range.
constexpr float kRebase = 8.0f;

// SUPER: 64-key tiles per LDS stage. The loads of a stage are issued together and waited for
// with one barrier, so a barrier falls on every SUPER-th step and a stage's loads are issued
// (STAGES - 2) * SUPER + 1 .. (STAGES - 1) * SUPER steps before its K fragments are read.
template <int D, int QT, int NW, int STAGES, int SUPER>
__global__ __launch_bounds__(NW * 64) void flash_kernel(FlashArgs a) {
  constexpr int DC = D / 16;             // k-steps of S
  constexpr int DT = D / 32;             // dim tiles of O
  constexpr int TILE = KB * D;           // halfs per K (or V) tile image
  constexpr int NSLOT = STAGES * SUPER;  // tile slots in LDS; tile t lives in slot t % NSLOT
  static_assert(STAGES == 3 || (STAGES == 4 && SUPER == 1), "three stages, or four of one tile");
  static_assert(SUPER == 1 || SUPER == 2, "one or two tiles per stage");

  // K of tile t+1 and V of tile t are read while the later stages land
  __shared__ __attribute__((aligned(16))) half_t ks[NSLOT][TILE];
  __shared__ __attribute__((aligned(16))) half_t vts[NSLOT][TILE];
  __shared__ __attribute__((aligned(16))) float kbias[NSLOT][KB];

  // Work unit: (pair = batch*H + head, query block). With xcd_order, consecutive block ids
  // land on different XCDs (round-robin dispatch), so block id i is mapped to pair
  // (i % 8) + 8 * ((i / 8) / qblocks): every query block of a pair runs on one XCD and its
  // K/V tiles are fetched into that XCD's L2 once.
  int pair, qb;
  {
    const int id = blockIdx.x;
    if (a.xcd_order) {
      const int local = id >> 3;
      pair = (id & 7) + 8 * (local / a.qblocks);
      qb = local % a.qblocks;
    } else {
      pair = id / a.qblocks;
      qb = id % a.qblocks;
    }
  }
  const int b = pair / a.H, h = pair % a.H, bh = pair;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qb * (NW * QT * 32) + wave * QT * 32;
  const int lq = lane & 31, hi = lane >> 5;
  const int ntiles = a.Lk_pad / KB;

  const half_t* Kt = a.Kc + (long long)bh * ntiles * TILE;
  const half_t* Vt = a.Vc + (long long)bh * ntiles * TILE;
  const float* Bg = a.bias2 + (long long)b * a.Lk_pad;

  half8_t qf[QT][DC];
  load_q<D, QT>(a, b, h, bh, q0, lq, hi, qf);

  float16_t o[QT][DT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qt][dt][r] = 0.f;
  float m_ref[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_ref[qt] = 0.f;
    l_run[qt] = 0.f;
  }

  TileLoader<D, NW> loader(Kt, Vt, Bg, lds_addr(ks), lds_addr(vts), lds_addr(kbias), wave, lane);
  auto dma = [&](int t, int st) { loader.issue(t, st); };
  auto wait_newer = [&](auto n_c) { loader.template wait_newer<decltype(n_c)::value>(); };
  using W0_ = std::integral_constant<int, 0>;
  using W1_ = std::integral_constant<int, 1>;
  using W2_ = std::integral_constant<int, 2>;

  // S^T = K Q^T - m_ref for the 64-key tile in LDS stage `buf`: the accumulators start at
  // -m_ref, so scores come out relative to the softmax reference (log2 units) and exp2 needs
  // no subtraction. s[kt][qt][r] = score(key 64t + 32kt + 8(r/4) + 4hi + r%4, query lq).
  // K fragment i = 2c + kt: chunk 2c + hi (dims 16c + 8hi .. +7) of key 32kt + lq.
  constexpr int NK = 2 * DC;  // K fragments (and score MFMA groups) per tile
  constexpr int NV = 4 * DT;  // V fragments (and output MFMA groups) per tile
  auto read_k = [&](int i, int buf) {
    const int c = i / 2, kt = i % 2;
    return *reinterpret_cast<const half8_t*>(&ks[buf][((2 * c + hi) * KB + kt * 32 + lq) * 8]);
  };
  // V fragment i = (2kt + kk) * DT + dt: stored key chunk 4kt + 2kk + hi of dim 32dt + lq
  auto read_v = [&](int i, int buf) {
    const int kt = i / (2 * DT), kk = (i / DT) % 2, dt = i % DT;
    return *reinterpret_cast<const half8_t*>(&vts[buf][((4 * kt + 2 * kk + hi) * D + dt * 32 + lq) * 8]);
  };
  // -m_ref in all 16 accumulator slots: the C operand of the first score MFMA of each chain
  // (rewritten only when the reference moves)
  float16_t minit[QT];
  auto set_minit = [&]() {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int r = 0; r < 16; ++r) minit[qt][r] = -m_ref[qt];
  };
  auto qk_mfma = [&](float16_t (&s)[2][QT], int i, const half8_t& kf) {
    const int c = i / 2, kt = i % 2;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
      s[kt][qt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[qt][c], c == 0 ? minit[qt] : s[kt][qt], 0, 0, 0);
  };
  // per-key bias of a tile (text and padding keys)
  auto add_bias = [&](float16_t (&s)[2][QT], int buf) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 bb = *reinterpret_cast<const float4*>(&kbias[buf][kt * 32 + 8 * g + 4 * hi]);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          s[kt][qt][4 * g + 0] += bb.x;
          s[kt][qt][4 * g + 1] += bb.y;
          s[kt][qt][4 * g + 2] += bb.z;
          s[kt][qt][4 * g + 3] += bb.w;
        }
      }
  };
  // partial row maximum over one 32-key half (kt) of the tile, 16 values per lane
  // (a tree of three-input maxima: dependency depth 3 instead of 15)
  auto half_max = [&](float16_t (&s)[2][QT], int kt, int qt) {
    const float16_t& v = s[kt][qt];
    const float a = __builtin_fmaxf(__builtin_fmaxf(v[0], v[1]), v[2]);
    const float b = __builtin_fmaxf(__builtin_fmaxf(v[3], v[4]), v[5]);
    const float c = __builtin_fmaxf(__builtin_fmaxf(v[6], v[7]), v[8]);
    const float d = __builtin_fmaxf(__builtin_fmaxf(v[9], v[10]), v[11]);
    const float e = __builtin_fmaxf(__builtin_fmaxf(v[12], v[13]), v[14]);
    return __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(a, b), c),
                           __builtin_fmaxf(__builtin_fmaxf(d, e), v[15]));
  };
  // maximum of a lane's value and the one 32 lanes away (the other half of the query column)
  auto col_max = [&](float m) {
    float lo = m, hi2 = m;
    permlane32_swap(lo, hi2);
    return __builtin_fmaxf(lo, hi2);
  };

  // Software pipeline, one barrier per tile. Step t:
  //   wait for this wave's loads of tile t+1, barrier (every wave's loads of tile t+1 have
  //   landed; every wave is done with step t-1), start loading tile t+STAGES-1 into the stage
  //   that held tile t-1;
  //   move the softmax reference if tile t needs it (rare);
  //   phase A: scores of tile t+1 on the MFMA pipe, K fragments read two MFMA groups ahead,
  //            the exp/convert/sum of tile t spread between the MFMA groups;
  //   phase B: O += V_t P_t on the MFMA pipe, V fragments read two MFMA groups ahead, the key
  //            bias (for the tiles that have one) and row max of tile t+1 between them.
  // Steps alternate the two score buffers (A holds tile t, B receives tile t+1).
  float16_t sA[2][QT], sB[2][QT];
  float mA[QT], mB[QT];
  const int issued = (STAGES - 1) * SUPER < ntiles ? (STAGES - 1) * SUPER : ntiles;
  for (int i = 0; i < issued; ++i) dma(i, i);
  {
    // the first stage (tiles 0 .. SUPER-1) has landed once at most the tiles issued after it
    // remain in flight
    const int newer = issued - (SUPER < ntiles ? SUPER : ntiles);
    if (newer >= 2) wait_newer(W2_{});
    else if (newer == 1) wait_newer(W1_{});
    else wait_newer(W0_{});
  }
  __syncthreads();
  set_minit();
#pragma unroll
  for (int i = 0; i < NK; ++i) qk_mfma(sA, i, read_k(i, 0));
  if (0 >= a.bias_block0) add_bias(sA, 0);

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float m = fmaxf(half_max(sA, 0, qt), half_max(sA, 1, qt));
    mA[qt] = col_max(m);
  }

  auto step = [&](int t, float16_t (&s_cur)[2][QT], float16_t (&s_nxt)[2][QT], float (&mx_cur)[QT],
                  float (&mx_nxt)[QT], auto more_c, auto bias_c, auto sync_c) {
    constexpr bool MORE = decltype(more_c)::value;
    constexpr bool BIAS = decltype(bias_c)::value;  // tile t+1 carries a key bias
    constexpr bool SYNC = decltype(sync_c)::value;  // t is the first tile of its stage
    const int vbuf = t % NSLOT, kbuf = (t + 1) % NSLOT;
    // On the first step of stage u: the next stage (which holds tile t+1 for SUPER = 1, and the
    // K of tile t+SUPER that step t+SUPER-1 reads) has landed once at most the tiles issued after
    // it remain in flight; the barrier then covers every wave's loads, and every wave's reads of
    // stage u-1, which the loads of stage u+STAGES-1 overwrite
    if (SYNC) {
      if (MORE && STAGES == 4 && t + 2 < ntiles) wait_newer(W1_{});
      else wait_newer(W0_{});
      __syncthreads();
      const int first = (t / SUPER + STAGES - 1) * SUPER;
#pragma unroll
      for (int r = 0; r < SUPER; ++r)
        if (MORE && first + r < ntiles) dma(first + r, (first + r) % NSLOT);
    }

    // ---- move the reference when a score exceeds it by more than 2^kRebase, or when nothing
    // has been accumulated yet (l = 0: the tile maximum becomes the reference, so the largest
    // p is 1 and l >= 1 afterwards); the running sum and output scale by 2^-shift and the
    // tile's relative scores drop by shift
    {
      bool need = false;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) need |= (mx_cur[qt] > kRebase) || (l_run[qt] == 0.f);
      if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float shift = (l_run[qt] == 0.f) ? mx_cur[qt] : fmaxf(mx_cur[qt], 0.f);
          const float alpha = __builtin_amdgcn_exp2f(-shift);
          m_ref[qt] += shift;
          l_run[qt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[qt][dt][r] *= alpha;
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) s_cur[kt][qt][r] -= shift;
        }
        set_minit();
      }
    }

    // ---- phase A; the scheduling barriers keep each phase's reads and VALU work inside the
    // phase
    __builtin_amdgcn_sched_barrier(0);
    // P of tile t in fp16, pair by pair: pair p = ((kt*QT + qt)*2 + kk)*4 + e/2
    constexpr int NP = 2 * QT * 2 * 4;
    half8_t pf[2][QT][2];
    float ls[2][QT];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) ls[kt][qt] = 0.f;
    auto exp_pair = [&](int p) {
      const int e = (p % 4) * 2, kk = (p / 4) % 2, qt = (p / 8) % QT, kt = p / (8 * QT);
      half2_t pp;
      pp[0] = (half_t)__builtin_amdgcn_exp2f(s_cur[kt][qt][kk * 8 + e]);
      pp[1] = (half_t)__builtin_amdgcn_exp2f(s_cur[kt][qt][kk * 8 + e + 1]);
      pf[kt][qt][kk][e] = pp[0];
      pf[kt][qt][kk][e + 1] = pp[1];
      const half2_t one = {(half_t)1.0f, (half_t)1.0f};
      ls[kt][qt] = __builtin_amdgcn_fdot2(pp, one, ls[kt][qt], false);
    };
    // The exp work is spread over both phases so that every MFMA slot carries a similar share
    // of VALU work (a wave issues its VALU work while its own MFMA runs, but only a short run of
    // it per MFMA hides): phase A takes the pairs of score half 0 and some of half 1, phase B's
    // first half (the MFMAs that consume P half 0) the rest of half 1.
    constexpr int PA_BAL = NP * NK / (NK + NV / 2);
    constexpr int PA = PA_BAL > NP / 2 ? PA_BAL : NP / 2;
    if (MORE) {
      // K fragment i+2 is read before the MFMAs of fragment i; each slot also does its share
      // of the exp work. Scheduling barriers pin this order (the default scheduler would put
      // every read right before its MFMA to save registers).
      half8_t kf[NK];
      kf[0] = read_k(0, kbuf);
      kf[1] = read_k(1, kbuf);
#pragma unroll
      for (int i = 0; i < NK; ++i) {
        if (i + 2 < NK) kf[i + 2] = read_k(i + 2, kbuf);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = i * PA / NK; p < (i + 1) * PA / NK; ++p) exp_pair(p);
        qk_mfma(s_nxt, i, kf[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int p = 0; p < PA; ++p) exp_pair(p);
    }

    __builtin_amdgcn_sched_barrier(0);
    // ---- phase B: O^T += V^T P^T, the DT accumulators interleaved. Slots 0 .. NV/2-1 use P of
    // score half 0 and finish the exp pairs of half 1; slots NV/2 .. NV-1 use half 1 and take
    // the key bias (for the tiles that have one) and the half-row maxima of tile t+1.
    {
      half8_t vf[NV];
      float hm[2][QT];
      vf[0] = read_v(0, vbuf);
      vf[1] = read_v(1, vbuf);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (i + 2 < NV) vf[i + 2] = read_v(i + 2, vbuf);
        __builtin_amdgcn_sched_barrier(0);
        const int kt = i / (2 * DT), kk = (i / DT) % 2, dt = i % DT;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          o[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i], pf[kt][qt][kk], o[qt][dt], 0, 0, 0);
        if (i < NV / 2) {
#pragma unroll
          for (int p = PA + i * (NP - PA) / (NV / 2); p < PA + (i + 1) * (NP - PA) / (NV / 2); ++p) exp_pair(p);
        } else if (MORE) {
          const int j = i - NV / 2;
          if (BIAS && j == 0) add_bias(s_nxt, kbuf);
          if (j < 2 * QT) {
            hm[j / QT][j % QT] = half_max(s_nxt, j / QT, j % QT);
            // keep the maximum in this slot (it would otherwise sink to its use after the loop)
            asm volatile("" : "+v"(hm[j / QT][j % QT]));
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (MORE) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          mx_nxt[qt] = col_max(fmaxf(hm[0][qt], hm[1][qt]));
        }
      }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) l_run[qt] += ls[0][qt] + ls[1][qt];
    __builtin_amdgcn_sched_barrier(0);
  };
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  // Steps before tb feed tiles without a key bias; tb is rounded down to even (adding the zero
  // bias of image keys is harmless) so the first loop ends on the A buffer.
  int tb = a.bias_block0 - 1;
  tb = tb < 0 ? 0 : (tb > ntiles - 1 ? ntiles - 1 : tb);
  tb &= ~1;
  // steps go in pairs from an even t, so with SUPER = 2 the first step of a pair starts a stage
  using S2_ = std::integral_constant<bool, SUPER == 1>;
  int t = 0;
  for (; t < tb; t += 2) {
    step(t, sA, sB, mA, mB, T_{}, F_{}, T_{});
    step(t + 1, sB, sA, mB, mA, T_{}, F_{}, S2_{});
  }
  for (; t + 2 < ntiles; t += 2) {
    step(t, sA, sB, mA, mB, T_{}, T_{}, T_{});
    step(t + 1, sB, sA, mB, mA, T_{}, T_{}, S2_{});
  }
  if (t + 1 < ntiles) {
    step(t, sA, sB, mA, mB, T_{}, T_{}, T_{});
    step(t + 1, sB, sA, mB, mA, F_{}, F_{}, S2_{});
  } else {
    step(t, sA, sB, mA, mB, F_{}, F_{}, T_{});
  }

  // ---- normalise and store: o[qt][dt][r] = O[query lq][dim dt*32 + 8(r/4) + 4hi + r%4]
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l_tot = l_run[qt] + __shfl_xor(l_run[qt], 32, 64);
    const float inv = 1.0f / l_tot;
    const int q = q0 + qt * 32 + lq;
    if (q >= a.Lq) continue;
    float* orow = a.O + a.oOff + (long long)b * a.oBatch + (long long)q * a.ldo + (long long)h * D + 4 * hi;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float4 v = make_float4(o[qt][dt][4 * g] * inv, o[qt][dt][4 * g + 1] * inv,
                               o[qt][dt][4 * g + 2] * inv, o[qt][dt][4 * g + 3] * inv);
        *reinterpret_cast<float4*>(orow + dt * 32 + 8 * g) = v;
      }
  }
}

// Wide variant for grids that fill the chip with 512-query blocks (the batch-2 CFG pair at
// 3952 x 4208: 8 query blocks x 32 (batch, head) pairs = 256 work-groups): every wave owns 64
// queries (two 32-query column tiles), so one 64-key K/V tile staged in LDS serves 512 queries
// and the copies and barriers per product are halved. The Q^T fragments no longer fit in
// registers beside the second tile's accumulators: the prologue writes each wave's prepared
// queries into its own chunk-major LDS region (chunk 2c + hi of query 32 qt + lq at
// (chunk * 64 + 32 qt + lq) * 8 halfs, conflict-free like K), and the score products read them
// back. One score buffer per step, K/V in two LDS stages:
//   barrier, copy tile t+1 -> QK of tile t (24 MFMAs) -> key bias, row maxima, lazy reference
//   move -> P = exp2(S) -> PV of tile t (24 MFMAs)
// Fragment reads are issued one k-step (QK) or two fragments (PV) ahead of their products; the
// scheduling barriers keep that order (the default scheduler would place every read right
// before its product). The softmax arithmetic, the lazy reference and the fp16 P with its row
// sums are those of flash_kernel, so the two give the same results.
template <int D>
__global__ __launch_bounds__(512) void flash_wide_kernel(FlashArgs a) {
  constexpr int NW = 8;          // waves per block
  constexpr int QT = 2;          // 32-query column tiles per wave
  constexpr int DC = D / 16;     // k-steps of S
  constexpr int DT = D / 32;     // dim tiles of O
  constexpr int TILE = KB * D;   // halfs per K (or V) tile image
  constexpr int QCH = D / 8;     // 8-dim chunks of a Q row
  __shared__ __attribute__((aligned(16))) half_t qs[NW][QCH * 64 * 8];
  __shared__ __attribute__((aligned(16))) half_t ks[2][TILE];
  __shared__ __attribute__((aligned(16))) half_t vts[2][TILE];
  __shared__ __attribute__((aligned(16))) float kbias[2][KB];

  int pair, qb;
  {
    const int id = blockIdx.x;
    if (a.xcd_order) {
      const int local = id >> 3;
      pair = (id & 7) + 8 * (local / a.qblocks);
      qb = local % a.qblocks;
    } else {
      pair = id / a.qblocks;
      qb = id % a.qblocks;
    }
  }
  const int b = pair / a.H, h = pair % a.H, bh = pair;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qb * (NW * QT * 32) + wave * QT * 32;
  const int lq = lane & 31, hi = lane >> 5;
  const int ntiles = a.Lk_pad / KB;

  const half_t* Kt = a.Kc + (long long)bh * ntiles * TILE;
  const half_t* Vt = a.Vc + (long long)bh * ntiles * TILE;
  const float* Bg = a.bias2 + (long long)b * a.Lk_pad;
  TileLoader<D, NW> loader(Kt, Vt, Bg, lds_addr(ks), lds_addr(vts), lds_addr(kbias), wave, lane);
  loader.issue(0, 0);
  if (ntiles > 1) loader.issue(1, 1);

  half_t* qw = &qs[wave][0];
  {
    half8_t qf[QT][DC];
    load_q<D, QT>(a, b, h, bh, q0, lq, hi, qf);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int c = 0; c < DC; ++c)
        *reinterpret_cast<half8_t*>(qw + ((2 * c + hi) * 64 + 32 * qt + lq) * 8) = qf[qt][c];
  }

  float16_t o[QT][DT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qt][dt][r] = 0.f;
  float m_ref[QT], l_run[QT];
  float16_t minit[QT];  // -m_ref in every accumulator slot: the C operand of each score chain
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_ref[qt] = 0.f;
    l_run[qt] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) minit[qt][r] = 0.f;
  }

  auto read_k = [&](int c, int kt, int buf) {
    return *reinterpret_cast<const half8_t*>(&ks[buf][((2 * c + hi) * KB + kt * 32 + lq) * 8]);
  };
  auto read_q = [&](int c, int qt) {
    return *reinterpret_cast<const half8_t*>(qw + ((2 * c + hi) * 64 + 32 * qt + lq) * 8);
  };
  // V fragment i = (2kt + kk) * DT + dt: stored key chunk 4kt + 2kk + hi of dim 32dt + lq
  auto read_v = [&](int i, int buf) {
    const int kt = i / (2 * DT), kk = (i / DT) % 2, dt = i % DT;
    return *reinterpret_cast<const half8_t*>(&vts[buf][((4 * kt + 2 * kk + hi) * D + dt * 32 + lq) * 8]);
  };
  auto half_max = [&](const float16_t& v) {
    const float a0 = __builtin_fmaxf(__builtin_fmaxf(v[0], v[1]), v[2]);
    const float b0 = __builtin_fmaxf(__builtin_fmaxf(v[3], v[4]), v[5]);
    const float c0 = __builtin_fmaxf(__builtin_fmaxf(v[6], v[7]), v[8]);
    const float d0 = __builtin_fmaxf(__builtin_fmaxf(v[9], v[10]), v[11]);
    const float e0 = __builtin_fmaxf(__builtin_fmaxf(v[12], v[13]), v[14]);
    return __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(a0, b0), c0),
                           __builtin_fmaxf(__builtin_fmaxf(d0, e0), v[15]));
  };
  auto col_max = [&](float m) {
    float lo = m, hi2 = m;
    permlane32_swap(lo, hi2);
    return __builtin_fmaxf(lo, hi2);
  };

  vm_wait<0>();
  __syncthreads();

  auto step = [&](int t, auto bias_c) {
    constexpr bool BIAS = decltype(bias_c)::value;
    const int buf = t & 1;
    // tile t landed (this wave's copies, then the barrier for every wave's); every wave is done
    // with tile t-1, whose stage now receives tile t+1
    if (t > 0) {
      vm_wait<0>();
      __syncthreads();
      if (t + 1 < ntiles) loader.issue(t + 1, buf ^ 1);
    }
    // ---- S^T = K Q^T - m_ref
    float16_t s[2][QT];
    {
      half8_t kf[2][2], qf[2][QT];
      kf[0][0] = read_k(0, 0, buf);
      kf[0][1] = read_k(0, 1, buf);
      qf[0][0] = read_q(0, 0);
      qf[0][1] = read_q(0, 1);
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const int cur = c & 1, nx = cur ^ 1;
        if (c + 1 < DC) {
          kf[nx][0] = read_k(c + 1, 0, buf);
          kf[nx][1] = read_k(c + 1, 1, buf);
          qf[nx][0] = read_q(c + 1, 0);
          qf[nx][1] = read_q(c + 1, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
            s[kt][qt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[cur][kt], qf[cur][qt], c == 0 ? minit[qt] : s[kt][qt],
                                                               0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (BIAS) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 bb = *reinterpret_cast<const float4*>(&kbias[buf][kt * 32 + 8 * g + 4 * hi]);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            s[kt][qt][4 * g + 0] += bb.x;
            s[kt][qt][4 * g + 1] += bb.y;
            s[kt][qt][4 * g + 2] += bb.z;
            s[kt][qt][4 * g + 3] += bb.w;
          }
        }
    }
    // ---- the reference moves when a score exceeds it by more than 2^kRebase, or on the first
    // tile (nothing accumulated yet: the reference becomes the tile maximum)
    {
      float mx[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) mx[qt] = col_max(__builtin_fmaxf(half_max(s[0][qt]), half_max(s[1][qt])));
      bool need = false;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) need |= (mx[qt] > kRebase) || (l_run[qt] == 0.f);
      if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float shift = (l_run[qt] == 0.f) ? mx[qt] : fmaxf(mx[qt], 0.f);
          const float alpha = __builtin_amdgcn_exp2f(-shift);
          m_ref[qt] += shift;
          l_run[qt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[qt][dt][r] *= alpha;
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kt][qt][r] -= shift;
#pragma unroll
          for (int r = 0; r < 16; ++r) minit[qt][r] = -m_ref[qt];
        }
      }
    }
    // ---- P = exp2(S) in fp16; row sums of the rounded values the PV products use
    half8_t pf[2][QT][2];
    {
      float ls[QT] = {0.f, 0.f};
      const half2_t one = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
              half2_t pp;
              pp[0] = (half_t)__builtin_amdgcn_exp2f(s[kt][qt][kk * 8 + e]);
              pp[1] = (half_t)__builtin_amdgcn_exp2f(s[kt][qt][kk * 8 + e + 1]);
              pf[kt][qt][kk][e] = pp[0];
              pf[kt][qt][kk][e + 1] = pp[1];
              ls[qt] = __builtin_amdgcn_fdot2(pp, one, ls[qt], false);
            }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) l_run[qt] += ls[qt];
    }
    // ---- O^T += V^T P^T
    {
      constexpr int NV = 4 * DT;
      half8_t vf[NV];
      vf[0] = read_v(0, buf);
      vf[1] = read_v(1, buf);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (i + 2 < NV) vf[i + 2] = read_v(i + 2, buf);
        __builtin_amdgcn_sched_barrier(0);
        const int kt = i / (2 * DT), kk = (i / DT) % 2, dt = i % DT;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          o[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i], pf[kt][qt][kk], o[qt][dt], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  // tiles before bias_block0 hold image keys only (no key bias)
  int tb = a.bias_block0;
  tb = tb < 0 ? 0 : (tb > ntiles ? ntiles : tb);
  int t = 0;
  for (; t < tb; ++t) step(t, F_{});
  for (; t < ntiles; ++t) step(t, T_{});

  // ---- normalise and store: o[qt][dt][r] = O[query 32 qt + lq][dim dt*32 + 8(r/4) + 4hi + r%4]
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l_tot = l_run[qt] + __shfl_xor(l_run[qt], 32, 64);
    const float inv = 1.0f / l_tot;
    const int q = q0 + qt * 32 + lq;
    if (q >= a.Lq) continue;
    float* orow = a.O + a.oOff + (long long)b * a.oBatch + (long long)q * a.ldo + (long long)h * D + 4 * hi;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float4 v = make_float4(o[qt][dt][4 * g] * inv, o[qt][dt][4 * g + 1] * inv, o[qt][dt][4 * g + 2] * inv,
                               o[qt][dt][4 * g + 3] * inv);
        *reinterpret_cast<float4*>(orow + dt * 32 + 8 * g) = v;
      }
  }
}

template <int D, int QT, int NW, int STAGES = 3, int SUPER = 1>
void launch_flash(FlashArgs fa, hipStream_t s) {
  constexpr int BQ = NW * QT * 32;
  fa.qblocks = (fa.Lq + BQ - 1) / BQ;
  const int blocks = fa.qblocks * fa.pairs;
  fa.xcd_order = (fa.pairs % 8 == 0) ? 1 : 0;
  flash_kernel<D, QT, NW, STAGES, SUPER><<<blocks, NW * 64, 0, s>>>(fa);
}

// The wide kernel where its grid of 512-query blocks covers every CU of the chip (D = 96: its
// queries, K and V stages need 148 KB of LDS and its accumulators 250 VGPRs); the 256-query
// kernel otherwise (the batch-1 DiT calls: 8 x 16 wide blocks would leave half the CUs idle).
// The wide kernel reads Q from the fp32 view (qraw), which masks rows past Lq; the packed Qp is
// padded to 256 rows only.
constexpr int kWideQueries = 512;
constexpr int kChipCUs = 256;

template <int D>
void launch_flash_auto(FlashArgs fa, hipStream_t s) {
  const int wide_blocks = (fa.Lq + kWideQueries - 1) / kWideQueries * fa.pairs;
  if (D == 96 && fa.qraw && wide_blocks >= kChipCUs) {
    fa.qblocks = (fa.Lq + kWideQueries - 1) / kWideQueries;
    fa.xcd_order = (fa.pairs % 8 == 0) ? 1 : 0;
    flash_wide_kernel<96><<<wide_blocks, 512, 0, s>>>(fa);
  } else {
    launch_flash<D, 1, 8>(fa, s);
  }
}

template <int D>
void launch_pack(const PackArgs& pa, int batch, bool vec, hipStream_t s) {
  const int rows = (pa.skip_q || pa.Lk_pad > pa.Lq_pad) ? pa.Lk_pad : pa.Lq_pad;
  if (vec) attn_pack_vec_kernel<D><<<dim3(rows / KB, pa.H, batch), 256, 0, s>>>(pa);
  else attn_pack_kernel<D><<<dim3(rows / KB, pa.H, batch), 256, 0, s>>>(pa);
}

// profile: bracket the two launches with the kernel profiler's events (off for the
// allocation-free entry point, whose callers may not create events)
template <int D>
int run_attention(PackArgs pa, FlashArgs fa, int batch, bool vec, bool profile) {
  hipStream_t s = ns2::stream();
  fa.pairs = pa.H * batch;
  if (!profile) {
    launch_pack<D>(pa, batch, vec, s);
    NS2_LAUNCHED("attn_pack");
    launch_flash_auto<D>(fa, s);
    NS2_LAUNCHED("attn_flash");
    return NS2_OK;
  }
  {
    ns2::ProfScope prof_("attn_pack");
    launch_pack<D>(pa, batch, vec, s);
    NS2_LAUNCHED("attn_pack");
  }
  ns2::ProfScope prof_("attn_flash");
  launch_flash_auto<D>(fa, s);
  NS2_LAUNCHED("attn_flash");
  return NS2_OK;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---- attention without the fused kernel's restrictions ---------------------------------------
//
// The semantics of ops.attention's materialized path (app/gpu/ops.js:211-241): causal masking,
// grouped K/V heads, any D <= 256, fp32 arithmetic. One wave per (query, head): lane l holds
// dims [DV l, DV l + DV) of q (pre-scaled by 1/sqrt(D)) and of the output row. Keys are taken
// four at a time (four independent dot products and wave sums in flight), with an online
// softmax. The waves of a block are the heads of one K/V group at one query, so they read the
// same K/V rows together and share them through L1.
struct RowsArgs {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  long long qOff, kOff, vOff;
  int Lq, Lk, H, D, ldq, ldk, ldv, ldo, group, causal, hpb;
  float scale;
};

template <int DV>
__global__ __launch_bounds__(1024) void attn_rows_kernel(RowsArgs a) {
  const int i = blockIdx.x;
  const int h = blockIdx.y * a.hpb + (threadIdx.x >> 6);
  if (h >= a.H) return;
  const int lane = threadIdx.x & 63;
  const int g = h / a.group;
  const int d0 = lane * DV;
  const float* qr = a.q + a.qOff + (long long)i * a.ldq + (long long)h * a.D;
  const float* kb = a.k + a.kOff + (long long)g * a.D;
  const float* vb = a.v + a.vOff + (long long)g * a.D;
  // lanes past D read element D - 1 (unconditional loads) with q = 0; their outputs are not stored
  float qv[DV], ov[DV];
  int dc[DV];
#pragma unroll
  for (int j = 0; j < DV; ++j) {
    dc[j] = d0 + j < a.D ? d0 + j : a.D - 1;
    qv[j] = d0 + j < a.D ? qr[dc[j]] * a.scale : 0.f;
    ov[j] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int kend = a.causal ? (i + 1 < a.Lk ? i + 1 : a.Lk) : a.Lk;
  auto dot = [&](int j) {
    const float* kr = kb + (long long)j * a.ldk;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < DV; ++e) s += qv[e] * kr[dc[e]];
    return s;
  };
  auto accumulate = [&](int j, float s) {
    const float mn = fmaxf(m, s);
    const float corr = __expf(m - mn), p = __expf(s - mn);
    l = l * corr + p;
    const float* vr = vb + (long long)j * a.ldv;
#pragma unroll
    for (int e = 0; e < DV; ++e) ov[e] = ov[e] * corr + p * vr[dc[e]];
    m = mn;
  };
  int j = 0;
  for (; j + 4 <= kend; j += 4) {
    float s0 = dot(j), s1 = dot(j + 1), s2 = dot(j + 2), s3 = dot(j + 3);
    s0 = wave_sum(s0);
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    s3 = wave_sum(s3);
    accumulate(j, s0);
    accumulate(j + 1, s1);
    accumulate(j + 2, s2);
    accumulate(j + 3, s3);
  }
  for (; j < kend; ++j) accumulate(j, wave_sum(dot(j)));
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  float* orow = a.o + (long long)i * a.ldo + (long long)h * a.D;
#pragma unroll
  for (int e = 0; e < DV; ++e)
    if (d0 + e < a.D) orow[d0 + e] = ov[e] * inv;
}

// The same attention on the matrix cores, for head dims D = 16 * DB with 16-byte aligned q, k
// and o views. A block of NW waves takes 16 queries of one head; wave w takes key blocks
// w, w + NW, ... (16 keys each), and the NW partial softmax states are merged through LDS at the
// end (flash-decoding style). The path is latency-bound at these sizes (a few hundred queries):
// splitting the keys over waves shortens each wave's chain of dependent loads, and each key
// block's K and V loads are issued together.
// Per key block the wave forms S^T = K Q^T (v_mfma_f32_16x16x16_f16, D/16 steps), whose
// accumulator layout is the B operand of O^T += V^T P^T, so probabilities never leave registers.
// Lane l holds query q0 + (l % 16): its scores for keys 4(l/16)..4(l/16)+3 of the block, and in
// product t (t < DB) the O^T rows r = 4(l/16) + j standing for d = DB r + t, which makes the
// online-softmax rescale a per-lane scalar, gives every lane DB consecutive d of a V row
// (vector loads) and makes its outputs one run of 4 DB consecutive d. Scores are in the log2
// domain (Q pre-scaled by log2(e)/sqrt(D)); fp16 operands, fp32 accumulation.
// At D = 256 a key row is 1 KB, one direct global->LDS copy: each wave copies its key block's
// 16 K rows into its own LDS rows (padded by 16 bytes, so the fragment reads of 16 rows hit 16
// different bank groups) and reads its K fragments from there. Every copy instruction moves
// 1 KB of consecutive bytes; the fragment loads straight from memory touched 16 rows per
// instruction and took 16.8 us against 13.2 us for the Gemma3 layer at 256 tokens.
constexpr int kRowsWaves = 8;  // waves per block of attn_rows_mfma_kernel (LDS: 8 * D * 64 B)

template <int DB, int NW>
__global__ __launch_bounds__(64 * NW) void attn_rows_mfma_kernel(RowsArgs a) {
  constexpr int D = 16 * DB;
  constexpr bool KDMA = D == 256;
  constexpr int RS = D * 4 + 16;                       // padded K row in LDS (bytes)
  constexpr int KST = KDMA ? 16 * RS : 0;              // K rows of one wave
  constexpr int OPB = NW * DB * 64 * 16;               // the partial outputs
  constexpr int SM = NW * KST > OPB ? NW * KST : OPB;  // K rows in the loop, then o_part
  __shared__ __attribute__((aligned(16))) char smem[SM];
  float4(*o_part)[DB][64] = reinterpret_cast<float4(*)[DB][64]>(smem);
  __shared__ float m_part[NW][16], l_part[NW][16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = blockIdx.y;
  // heaviest causal tiles first
  const int q0 = (gridDim.x - 1 - blockIdx.x) * 16;
  const int col = lane & 15, grp = lane >> 4;
  const int g = h / a.group;
  const int qi = q0 + col;
  const bool qvalid = qi < a.Lq;

  // Q^T fragments (the B operand of every S^T product), shared by the block's waves through
  // LDS; wave w converts fragments t = w, w + NW, ... Rows past the end are read from the last
  // row (loads stay unconditional, so they issue back to back); their scores are masked and
  // their probabilities are zero.
  __shared__ half4_t q_lds[DB][64];
  {
    const float* qr = a.q + a.qOff + (long long)(qvalid ? qi : a.Lq - 1) * a.ldq + (long long)h * D + 4 * grp;
    for (int t = wave; t < DB; t += NW) {
      const float4 x = *reinterpret_cast<const float4*>(qr + 16 * t);
      q_lds[t][lane] = half4_t{(half_t)(x.x * a.scale), (half_t)(x.y * a.scale), (half_t)(x.z * a.scale),
                               (half_t)(x.w * a.scale)};
    }
  }
  __syncthreads();
  const float* kb0 = a.k + a.kOff + (long long)g * D;
  const float* vb0 = a.v + a.vOff + (long long)g * D;

  float4_t o[DB];
#pragma unroll
  for (int t = 0; t < DB; ++t) o[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  const int qlast = (q0 + 15 < a.Lq ? q0 + 15 : a.Lq - 1);
  int nkb = (a.Lk + 15) / 16;
  if (a.causal && qlast / 16 + 1 < nkb) nkb = qlast / 16 + 1;
  for (int kb = wave; kb < nkb; kb += NW) {
    // keeps the Q^T fragments in LDS instead of 2 * DB registers hoisted out of the loop
    asm volatile("" ::: "memory");
    // K rows (key kb*16 + col) for S^T's A operand, and V^T (d = 16t + col, keys key0..key0+3)
    // for the PV product's A operand: all loads of the block issued before any use
    const int kr = kb * 16 + col;
    const int key0 = kb * 16 + 4 * grp;
    float4 kx[DB];
    if constexpr (KDMA) {
      const uint32_t kst = lds_addr(smem) + wave * KST;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * 16 + r;
        dma16(kb0 + (long long)(key < a.Lk ? key : a.Lk - 1) * a.ldk + 4 * lane,
              __builtin_amdgcn_readfirstlane(kst + r * RS));
      }
    } else {
      const float* krow = kb0 + (long long)(kr < a.Lk ? kr : a.Lk - 1) * a.ldk + 4 * grp;
#pragma unroll
      for (int t = 0; t < DB; ++t) kx[t] = *reinterpret_cast<const float4*>(krow + 16 * t);
    }
    // V^T's A operand in product t: row col = d DB col + t, keys key0 + j
    float vx[DB][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float* vr = vb0 + DB * col + (long long)(key0 + j < a.Lk ? key0 + j : a.Lk - 1) * a.ldv;
      if constexpr (DB % 4 == 0) {
#pragma unroll
        for (int t4 = 0; t4 < DB; t4 += 4) {
          const float4 x = *reinterpret_cast<const float4*>(vr + t4);
          vx[t4][j] = x.x;
          vx[t4 + 1][j] = x.y;
          vx[t4 + 2][j] = x.z;
          vx[t4 + 3][j] = x.w;
        }
      } else {
#pragma unroll
        for (int t = 0; t < DB; ++t) vx[t][j] = vr[t];
      }
    }
    // keep every load of the block in flight before the first use (left alone, the scheduler
    // converts each group of V values as it arrives and waits on each group in turn)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (KDMA) {
      // this wave's K rows have landed (it alone reads them): the fragments from LDS
      vm_wait<0>();
      asm volatile("" ::: "memory");
      const char* kst_p = smem + wave * KST;
#pragma unroll
      for (int t = 0; t < DB; ++t) kx[t] = *reinterpret_cast<const float4*>(kst_p + col * RS + (16 * t + 4 * grp) * 4);
    }
    float4_t s = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < DB; ++t) {
      const half4_t kf = half4_t{(half_t)kx[t].x, (half_t)kx[t].y, (half_t)kx[t].z, (half_t)kx[t].w};
      s = __builtin_amdgcn_mfma_f32_16x16x16f16(kf, q_lds[t][lane], s, 0, 0, 0);
    }
    // s[j]: key kb*16 + 4 grp + j of query qi
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = key0 + j;
      if (key >= a.Lk || (a.causal && key > qi)) s[j] = -INFINITY;
      bm = fmaxf(bm, s[j]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    // a block of a later wave may have no visible key for this query yet: keep the state
    // unchanged then (bm = -inf), instead of exp2(-inf - -inf)
    const float mn = fmaxf(m, bm);
    const float corr = mn == -INFINITY ? 1.f : exp2f(m - mn);
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = mn == -INFINITY ? 0.f : exp2f(s[j] - mn);
    lsum = lsum * corr + ((p[0] + p[1]) + (p[2] + p[3]));
    m = mn;
    const half4_t pf = half4_t{(half_t)p[0], (half_t)p[1], (half_t)p[2], (half_t)p[3]};
    // O^T += V^T P^T
#pragma unroll
    for (int t = 0; t < DB; ++t) {
      const half4_t vf = half4_t{(half_t)vx[t][0], (half_t)vx[t][1], (half_t)vx[t][2], (half_t)vx[t][3]};
      o[t] *= corr;
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, pf, o[t], 0, 0, 0);
    }
  }
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  if constexpr (KDMA) __syncthreads();  // every wave is done with its K rows (o_part overlays them)

  // merge the waves' states: O = sum_w 2^(m_w - M) O_w, L = sum_w 2^(m_w - M) l_w
#pragma unroll
  for (int t = 0; t < DB; ++t) o_part[wave][t][lane] = make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
  if (grp == 0) {
    m_part[wave][col] = m;
    l_part[wave][col] = lsum;
  }
  __syncthreads();
  if (!qvalid) return;
  float M = m_part[0][col];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, m_part[w][col]);  // finite: wave 0 sees key 0
  float sc[NW], L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    sc[w] = exp2f(m_part[w][col] - M);
    L += sc[w] * l_part[w][col];
  }
  const float inv = 1.0f / L;
  // the lane's outputs are d = 4 DB grp + f, f = DB j + t < 4 DB; wave w writes f in
  // [w FW, (w + 1) FW)
  constexpr int F = 4 * DB, FW = (F + NW - 1) / NW;
  float* orow = a.o + (long long)qi * a.ldo + (long long)h * D + F * grp;
#pragma unroll
  for (int u = 0; u < FW; ++u) {
    const int f = wave * FW + u;
    if (f < F) {
      const int j = f / DB, t = f % DB;
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) r += sc[w] * reinterpret_cast<const float*>(&o_part[w][t][lane])[j];
      orow[f] = r * inv;
    }
  }
}

// attn_rows_mfma_kernel with K and V stored as fp16 (the values its fp32 path converts before
// every product, so the results are the same bit for bit): half the bytes per key, and each
// wave issues the loads of two of its key blocks (kb and kb + NW) before it uses either, so a
// query block at a few hundred keys costs one round trip to memory instead of two. The blocks
// are then consumed in the order of the fp32 kernel, so every wave's online softmax sees the
// same sequence. At D = 256 the K rows go through LDS: one direct copy of 512 bytes (32 lanes)
// per key row, rows padded by 16 bytes, so the 8-byte fragment reads of 16 rows by 32 lanes fall
// in 64 different banks.
struct RowsArgsH {
  const float* q;
  const half_t* k;
  const half_t* v;
  float* o;
  long long qOff, kOff, vOff;  // k, v offsets and strides in fp16 elements
  int Lq, Lk, H, D, ldq, ldk, ldv, ldo, group, causal;
  float scale;
  // OPROJ: the output projection's share of each head instead of o (see attn_rows_h_kernel)
  const half_t* wo;  // fp16 weight tiles of W_o [N][H*D] (tile_w16_kernel's layout)
  float* part;       // [H][Lq][N] fp32
  int N;
  int ncs;           // OPROJ: blocks per (query block, head), blockIdx.z, each a range of N's 16-column tiles
};

// OPROJ: the block goes on from its normalized output O_h (16 queries x D of head h, rounded to
// fp16 as a linear's loader rounds its input) to O_h W_o[:, hD:(h+1)D]^T, head h's share of
// the output projection, into part[h] (16 x N, fp32): the projection split over heads, its H
// shares summed by the reduction that follows it, as a split-K linear's k-range shares are.
// Each wave takes 16-column tiles n0 = 16w, 16(w + NW), ... with v_mfma_f32_16x16x16_f16: A = O_h
// rows from LDS (row padded by 16 bytes), B = 4 consecutive k of weight row n0 + l%16 (8 bytes of
// one tile chunk). With ncs > 1, block z of a (query block, head) takes the z-th of ncs ranges of
// the column tiles (and repeats the attention): the grid fills CUs the attention alone leaves
// idle, and each block streams 1/ncs of the head's W_o slice.
template <int DB, int NW, bool OPROJ = false>
__global__ __launch_bounds__(64 * NW) void attn_rows_h_kernel(RowsArgsH a) {
  constexpr int D = 16 * DB;
  constexpr bool KDMA = D == 256;
  constexpr int RS = D * 2 + 16;                       // padded fp16 K row in LDS (bytes)
  constexpr int KST = KDMA ? 2 * 16 * RS : 0;          // K rows of one wave's two key blocks
  constexpr int OPB = NW * DB * 64 * 16;               // the partial outputs
  constexpr int SM = NW * KST > OPB ? NW * KST : OPB;  // K rows in the loop, then o_part
  __shared__ __attribute__((aligned(16))) char smem[SM];
  float4(*o_part)[DB][64] = reinterpret_cast<float4(*)[DB][64]>(smem);
  __shared__ float m_part[NW][16], l_part[NW][16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = blockIdx.y;
  const int q0 = (gridDim.x - 1 - blockIdx.x) * 16;
  const int col = lane & 15, grp = lane >> 4;
  const int g = h / a.group;
  const int qi = q0 + col;
  const bool qvalid = qi < a.Lq;

  __shared__ half4_t q_lds[DB][64];
  {
    const float* qr = a.q + a.qOff + (long long)(qvalid ? qi : a.Lq - 1) * a.ldq + (long long)h * D + 4 * grp;
    for (int t = wave; t < DB; t += NW) {
      const float4 x = *reinterpret_cast<const float4*>(qr + 16 * t);
      q_lds[t][lane] = half4_t{(half_t)(x.x * a.scale), (half_t)(x.y * a.scale), (half_t)(x.z * a.scale),
                               (half_t)(x.w * a.scale)};
    }
  }
  __syncthreads();
  const half_t* kb0 = a.k + a.kOff + (long long)g * D;
  const half_t* vb0 = a.v + a.vOff + (long long)g * D;

  float4_t o[DB];
#pragma unroll
  for (int t = 0; t < DB; ++t) o[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  const int qlast = (q0 + 15 < a.Lq ? q0 + 15 : a.Lq - 1);
  int nkb = (a.Lk + 15) / 16;
  if (a.causal && qlast / 16 + 1 < nkb) nkb = qlast / 16 + 1;

  // the loads of key block kb into slot u: K rows (LDS at D = 256, else registers) and the V^T
  // operand values (row col: d = DB col + t of keys key0 + j)
  auto load = [&](int kb, int u, half4_t (&kx)[DB], half_t (&vh)[4][DB]) {
    if constexpr (KDMA) {
      const uint32_t kst = lds_addr(smem) + wave * KST + u * 16 * RS;
      if (lane < D / 8) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * 16 + r;
          dma16(kb0 + (long long)(key < a.Lk ? key : a.Lk - 1) * a.ldk + 8 * lane,
                __builtin_amdgcn_readfirstlane(kst + r * RS));
        }
      }
    } else {
      const int kr = kb * 16 + col;
      const half_t* krow = kb0 + (long long)(kr < a.Lk ? kr : a.Lk - 1) * a.ldk + 4 * grp;
#pragma unroll
      for (int t = 0; t < DB; ++t) kx[t] = *reinterpret_cast<const half4_t*>(krow + 16 * t);
    }
    const int key0 = kb * 16 + 4 * grp;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half_t* vr = vb0 + DB * col + (long long)(key0 + j < a.Lk ? key0 + j : a.Lk - 1) * a.ldv;
      if constexpr (DB % 8 == 0) {
#pragma unroll
        for (int t8 = 0; t8 < DB; t8 += 8) {
          const half8_t x = *reinterpret_cast<const half8_t*>(vr + t8);
#pragma unroll
          for (int e = 0; e < 8; ++e) vh[j][t8 + e] = x[e];
        }
      } else if constexpr (DB % 4 == 0) {
#pragma unroll
        for (int t4 = 0; t4 < DB; t4 += 4) {
          const half4_t x = *reinterpret_cast<const half4_t*>(vr + t4);
#pragma unroll
          for (int e = 0; e < 4; ++e) vh[j][t4 + e] = x[e];
        }
      } else {
#pragma unroll
        for (int t = 0; t < DB; ++t) vh[j][t] = vr[t];
      }
    }
  };
  // one key block's scores, softmax update and PV products (the arithmetic of the fp32 kernel)
  auto consume = [&](int kb, int u, half4_t (&kx)[DB], const half_t (&vh)[4][DB]) {
    if constexpr (KDMA) {
      const char* kst_p = smem + wave * KST + u * 16 * RS;
#pragma unroll
      for (int t = 0; t < DB; ++t) kx[t] = *reinterpret_cast<const half4_t*>(kst_p + col * RS + (16 * t + 4 * grp) * 2);
    }
    float4_t s = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < DB; ++t) s = __builtin_amdgcn_mfma_f32_16x16x16f16(kx[t], q_lds[t][lane], s, 0, 0, 0);
    const int key0 = kb * 16 + 4 * grp;
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = key0 + j;
      if (key >= a.Lk || (a.causal && key > qi)) s[j] = -INFINITY;
      bm = fmaxf(bm, s[j]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float mn = fmaxf(m, bm);
    const float corr = mn == -INFINITY ? 1.f : exp2f(m - mn);
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = mn == -INFINITY ? 0.f : exp2f(s[j] - mn);
    lsum = lsum * corr + ((p[0] + p[1]) + (p[2] + p[3]));
    m = mn;
    const half4_t pf = half4_t{(half_t)p[0], (half_t)p[1], (half_t)p[2], (half_t)p[3]};
#pragma unroll
    for (int t = 0; t < DB; ++t) {
      const half4_t vf = half4_t{vh[0][t], vh[1][t], vh[2][t], vh[3][t]};
      o[t] *= corr;
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, pf, o[t], 0, 0, 0);
    }
  };

  for (int kb = wave; kb < nkb; kb += 2 * NW) {
    asm volatile("" ::: "memory");
    const bool two = kb + NW < nkb;  // uniform per wave
    half4_t kx0[DB], kx1[DB];
    half_t vh0[4][DB], vh1[4][DB];
    load(kb, 0, kx0, vh0);
    if (two) load(kb + NW, 1, kx1, vh1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (KDMA) {
      // this wave's K rows have landed (it alone reads them)
      vm_wait<0>();
      asm volatile("" ::: "memory");
    }
    consume(kb, 0, kx0, vh0);
    if (two) consume(kb + NW, 1, kx1, vh1);
  }
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  // OPROJ: the weight fragments of the wave's first JC column tiles are loaded here, so that
  // their latency passes during the merge (they do not depend on the attention)
  constexpr int JC = !OPROJ ? 1 : (DB == 14 || DB == 15) ? 1 : DB == 16 ? 5 : 3;
  half4_t bf[JC][DB];
  const int nt = OPROJ ? a.N / 16 : 0;
  const int j_lo = OPROJ ? (int)blockIdx.z * nt / a.ncs : 0, j_hi = OPROJ ? ((int)blockIdx.z + 1) * nt / a.ncs : 0;
  auto load_w = [&](int j0) {
#pragma unroll
    for (int c = 0; c < JC; ++c) {
      const int j = j0 + c * NW;
      if (j < j_hi) {  // uniform per wave
        const int n = 16 * j + col;
#pragma unroll
        for (int t = 0; t < DB; ++t)
          bf[c][t] = *reinterpret_cast<const half4_t*>(a.wo + tiled_off(n, h * D + 16 * t + 4 * grp, a.H * D));
      }
    }
  };
  if constexpr (OPROJ) load_w(j_lo + wave);
  if constexpr (KDMA) __syncthreads();  // every wave is done with its K rows (o_part overlays them)

#pragma unroll
  for (int t = 0; t < DB; ++t) o_part[wave][t][lane] = make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
  if (grp == 0) {
    m_part[wave][col] = m;
    l_part[wave][col] = lsum;
  }
  __syncthreads();
  if (!OPROJ && !qvalid) return;
  // (rows past Lq repeat row Lq - 1's state: finite, and only OPROJ computes them)
  float M = m_part[0][col];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, m_part[w][col]);  // finite: wave 0 sees key 0
  float sc[NW], L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    sc[w] = exp2f(m_part[w][col] - M);
    L += sc[w] * l_part[w][col];
  }
  const float inv = 1.0f / L;
  constexpr int F = 4 * DB, FW = (F + NW - 1) / NW;
  float res[FW];
#pragma unroll
  for (int u = 0; u < FW; ++u) {
    const int f = wave * FW + u;
    res[u] = 0.f;
    if (f < F) {
      const int j = f / DB, t = f % DB;
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) r += sc[w] * reinterpret_cast<const float*>(&o_part[w][t][lane])[j];
      res[u] = r * inv;
    }
  }
  if constexpr (!OPROJ) {
    float* orow = a.o + (long long)qi * a.ldo + (long long)h * D + F * grp;
#pragma unroll
    for (int u = 0; u < FW; ++u)
      if (wave * FW + u < F) orow[wave * FW + u] = res[u];
  } else {
    constexpr int OS = D + 8;  // fp16 row of O_h in LDS (16 bytes of padding)
    half_t* o16 = reinterpret_cast<half_t*>(smem);
    static_assert(16 * OS * 2 <= SM, "O_h fits the LDS of the loop");
    __syncthreads();  // every wave is done reading o_part
    if constexpr (FW == 8 && F % 8 == 0) {
      // one 16-byte store: the row stride (2D + 16 bytes) and F grp + 8 wave keep it aligned
      half8_t hv;
#pragma unroll
      for (int u = 0; u < 8; ++u) hv[u] = (half_t)res[u];
      *reinterpret_cast<half8_t*>(o16 + col * OS + F * grp + wave * FW) = hv;
    } else {
#pragma unroll
      for (int u = 0; u < FW; ++u)
        if (wave * FW + u < F) o16[col * OS + F * grp + wave * FW + u] = (half_t)res[u];
    }
    __syncthreads();
    half4_t af[DB];
#pragma unroll
    for (int t = 0; t < DB; ++t) af[t] = *reinterpret_cast<const half4_t*>(o16 + col * OS + 16 * t + 4 * grp);
    // the weight fragments of JC column tiles are loaded together (one round trip per JC tiles;
    // one tile at a time where the loop's K/V registers leave no room: D = 224, 240)
    for (int j0 = j_lo + wave; j0 < j_hi; j0 += JC * NW) {
      if (j0 != j_lo + wave) load_w(j0);
#pragma unroll
      for (int c = 0; c < JC; ++c) {
        const int j = j0 + c * NW;
        if (j < j_hi) {
          float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < DB; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x16f16(af[t], bf[c][t], acc, 0, 0, 0);
          // acc[i]: query q0 + 4 grp + i, column 16 j + col
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int q = q0 + 4 * grp + i;
            if (q < a.Lq) a.part[((long long)h * a.Lq + q) * a.N + 16 * j + col] = acc[i];
          }
        }
      }
    }
  }
}

}  // namespace

extern "C" int ns2_attention_rows(const float* q, const float* k, const float* v, float* o, int Lq, int Lk,
                                  int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff,
                                  long long kOff, long long vOff, int group, int causal) {
  NS2_READY();
  if (Lq <= 0 || H <= 0) return NS2_OK;
  NS2_REQUIRE(q && k && v && o, "ns2_attention_rows: null q, k, v or o");
  NS2_REQUIRE(D > 0 && D <= 256, "ns2_attention_rows: unsupported head dim %d", D);
  NS2_REQUIRE(group > 0 && H % group == 0, "ns2_attention_rows: H=%d is not a multiple of group=%d", H, group);
  NS2_REQUIRE(Lk > 0 && ldq >= H * D && ldk >= H / group * D && ldv >= H / group * D && ldo >= H * D && qOff >= 0 &&
                  kOff >= 0 && vOff >= 0,
              "ns2_attention_rows: bad sizes or strides");
  // the waves of a block: the heads of one K/V group (at most 16)
  const int hpb = group < 16 ? group : 16;
  RowsArgs a{q, k, v, o, qOff, kOff, vOff, Lq, Lk, H, D, ldq, ldk, ldv, ldo, group, causal ? 1 : 0, hpb,
             1.0f / sqrtf((float)D)};
  ns2::ProfScope prof_("attn_rows");
  hipStream_t s = ns2::stream();
  // matrix-core path: D a multiple of 16 and every row read or written 16-byte aligned
  auto al4 = [](long long x) { return x % 4 == 0; };
  const bool al = aligned16(q) && aligned16(k) && aligned16(v) && al4(ldq) && al4(ldk) && al4(ldv) &&
                  al4(qOff) && al4(kOff) && al4(vOff) && D % 16 == 0;
  if (al) {
    a.scale *= kLog2e;
    const dim3 mgrid((Lq + 15) / 16, H);
    switch (D / 16) {
#define NS2_ROWS_CASE(N) \
  case N: attn_rows_mfma_kernel<N, kRowsWaves><<<mgrid, 64 * kRowsWaves, 0, s>>>(a); break;
      NS2_ROWS_CASE(1) NS2_ROWS_CASE(2) NS2_ROWS_CASE(3) NS2_ROWS_CASE(4) NS2_ROWS_CASE(5) NS2_ROWS_CASE(6)
      NS2_ROWS_CASE(7) NS2_ROWS_CASE(8) NS2_ROWS_CASE(9) NS2_ROWS_CASE(10) NS2_ROWS_CASE(11)
      NS2_ROWS_CASE(12) NS2_ROWS_CASE(13) NS2_ROWS_CASE(14) NS2_ROWS_CASE(15) NS2_ROWS_CASE(16)
#undef NS2_ROWS_CASE
      default: break;
    }
    NS2_LAUNCHED("attn_rows_mfma");
    return NS2_OK;
  }
  const dim3 grid(Lq, (H + hpb - 1) / hpb), block(64 * hpb);
  const int dv = (D + 63) / 64;
  if (dv == 1) attn_rows_kernel<1><<<grid, block, 0, s>>>(a);
  else if (dv == 2) attn_rows_kernel<2><<<grid, block, 0, s>>>(a);
  else if (dv == 3) attn_rows_kernel<3><<<grid, block, 0, s>>>(a);
  else attn_rows_kernel<4><<<grid, block, 0, s>>>(a);
  NS2_LAUNCHED("attn_rows");
  return NS2_OK;
}

extern "C" int ns2_attention_rows_f16kv_oproj(const float* q, const uint16_t* k, const uint16_t* v,
                                              const uint16_t* wo_tiled, float* part, int Lq, int Lk, int H, int D,
                                              int ldq, int ldk, int ldv, long long qOff, long long kOff,
                                              long long vOff, int group, int causal, int N) {
  NS2_READY();
  if (Lq <= 0 || H <= 0) return NS2_OK;
  const char* fn = "ns2_attention_rows_f16kv_oproj";
  NS2_REQUIRE(q && k && v && wo_tiled && part, "%s: null q, k, v, wo_tiled or part", fn);
  NS2_REQUIRE(D > 0 && D <= 256 && D % 16 == 0, "%s: head dim %d is not a multiple of 16 up to 256", fn, D);
  NS2_REQUIRE(group > 0 && H % group == 0, "%s: H=%d is not a multiple of group=%d", fn, H, group);
  NS2_REQUIRE(N > 0 && N % 64 == 0 && (H * D) % 64 == 0,
              "%s: N=%d and H*D=%d must be multiples of 64 (the weight tiles)", fn, N, H * D);
  NS2_REQUIRE(Lk > 0 && ldq >= H * D && ldk >= H / group * D && ldv >= H / group * D && qOff >= 0 && kOff >= 0 &&
                  vOff >= 0,
              "%s: bad sizes or strides", fn);
  NS2_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(wo_tiled) && ldq % 4 == 0 &&
                  qOff % 4 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && kOff % 8 == 0 && vOff % 8 == 0,
              "%s: q, k, v rows and the weight tiles must be 16-byte aligned", fn);
  RowsArgsH a{q, reinterpret_cast<const half_t*>(k), reinterpret_cast<const half_t*>(v), nullptr, qOff, kOff, vOff,
              Lq, Lk, H, D, ldq, ldk, ldv, 0, group, causal ? 1 : 0, 1.0f / sqrtf((float)D) * kLog2e,
              reinterpret_cast<const half_t*>(wo_tiled), part, N, 1};
  // column ranges per (query block, head): up to 4, while the grid stays within one block per CU
  // (256 tokens, 4 heads: 64 -> 256 blocks)
  const int units = (Lq + 15) / 16 * H;
  while (a.ncs < 4 && units * a.ncs * 2 <= kChipCUs && N / 16 >= a.ncs * 2) a.ncs *= 2;
  ns2::ProfScope prof_("attn_rows_oproj");
  hipStream_t s = ns2::stream();
  const dim3 grid((Lq + 15) / 16, H, a.ncs);
  switch (D / 16) {
#define NS2_ROWS_HO_CASE(N_) \
  case N_: attn_rows_h_kernel<N_, kRowsWaves, true><<<grid, 64 * kRowsWaves, 0, s>>>(a); break;
    NS2_ROWS_HO_CASE(1) NS2_ROWS_HO_CASE(2) NS2_ROWS_HO_CASE(3) NS2_ROWS_HO_CASE(4) NS2_ROWS_HO_CASE(5)
    NS2_ROWS_HO_CASE(6) NS2_ROWS_HO_CASE(7) NS2_ROWS_HO_CASE(8) NS2_ROWS_HO_CASE(9) NS2_ROWS_HO_CASE(10)
    NS2_ROWS_HO_CASE(11) NS2_ROWS_HO_CASE(12) NS2_ROWS_HO_CASE(13) NS2_ROWS_HO_CASE(14) NS2_ROWS_HO_CASE(15)
    NS2_ROWS_HO_CASE(16)
#undef NS2_ROWS_HO_CASE
    default: break;
  }
  NS2_LAUNCHED("attn_rows_oproj");
  return NS2_OK;
}

extern "C" int ns2_attention_rows_f16kv(const float* q, const uint16_t* k, const uint16_t* v, float* o, int Lq,
                                        int Lk, int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff,
                                        long long kOff, long long vOff, int group, int causal) {
  NS2_READY();
  if (Lq <= 0 || H <= 0) return NS2_OK;
  NS2_REQUIRE(q && k && v && o, "ns2_attention_rows_f16kv: null q, k, v or o");
  NS2_REQUIRE(D > 0 && D <= 256 && D % 16 == 0, "ns2_attention_rows_f16kv: head dim %d is not a multiple of 16 up to 256",
              D);
  NS2_REQUIRE(group > 0 && H % group == 0, "ns2_attention_rows_f16kv: H=%d is not a multiple of group=%d", H, group);
  NS2_REQUIRE(Lk > 0 && ldq >= H * D && ldk >= H / group * D && ldv >= H / group * D && ldo >= H * D && qOff >= 0 &&
                  kOff >= 0 && vOff >= 0,
              "ns2_attention_rows_f16kv: bad sizes or strides");
  // 16-byte rows: q as fp32 (strides and offset multiples of 4), k and v as fp16 (multiples of 8)
  NS2_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && ldq % 4 == 0 && qOff % 4 == 0 && ldk % 8 == 0 &&
                  ldv % 8 == 0 && kOff % 8 == 0 && vOff % 8 == 0,
              "ns2_attention_rows_f16kv: q, k and v rows must be 16-byte aligned");
  RowsArgsH a{q, reinterpret_cast<const half_t*>(k), reinterpret_cast<const half_t*>(v), o, qOff, kOff, vOff, Lq, Lk,
              H, D, ldq, ldk, ldv, ldo, group, causal ? 1 : 0, 1.0f / sqrtf((float)D) * kLog2e};
  ns2::ProfScope prof_("attn_rows");
  hipStream_t s = ns2::stream();
  const dim3 grid((Lq + 15) / 16, H);
  switch (D / 16) {
#define NS2_ROWS_H_CASE(N) \
  case N: attn_rows_h_kernel<N, kRowsWaves><<<grid, 64 * kRowsWaves, 0, s>>>(a); break;
    NS2_ROWS_H_CASE(1) NS2_ROWS_H_CASE(2) NS2_ROWS_H_CASE(3) NS2_ROWS_H_CASE(4) NS2_ROWS_H_CASE(5)
    NS2_ROWS_H_CASE(6) NS2_ROWS_H_CASE(7) NS2_ROWS_H_CASE(8) NS2_ROWS_H_CASE(9) NS2_ROWS_H_CASE(10)
    NS2_ROWS_H_CASE(11) NS2_ROWS_H_CASE(12) NS2_ROWS_H_CASE(13) NS2_ROWS_H_CASE(14) NS2_ROWS_H_CASE(15)
    NS2_ROWS_H_CASE(16)
#undef NS2_ROWS_H_CASE
    default: break;
  }
  NS2_LAUNCHED("attn_rows_h");
  return NS2_OK;
}

namespace {

// The body of ns2_attention and ns2_attention_noalloc: the packed operands live in library
// workspace, or (noalloc) are carved from the fixed scratch array.
int attention_call(const char* fn, bool noalloc, const float* q, const float* k, const float* v, float* o,
                   int batch, int Lq, int Lk, int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff,
                   long long kOff, long long vOff, long long oOff, long long qBatch, long long kBatch,
                   long long vBatch, long long oBatch, float scale, const float* key_bias, int biasStart,
                   long long biasBatch, const float* q_norm, const float* k_norm, float eps,
                   const float* rope_cs, long long sin_off, int rope_rows, const float* k_text = nullptr,
                   const float* v_text = nullptr, int ld_text = 0, int text_start = 0, uint16_t* vpk = nullptr,
                   int v_rows = 0) {
  NS2_READY();
  if (Lq <= 0 || batch <= 0) return NS2_OK;
  NS2_REQUIRE(q && k && v && o, "%s: null q, k, v or o", fn);
  NS2_REQUIRE(D == 32 || D == 64 || D == 96 || D == 128, "%s: unsupported head dim %d", fn, D);
  NS2_REQUIRE(Lk > 0 && H > 0, "%s: Lk=%d H=%d", fn, Lk, H);
  NS2_REQUIRE(ldo % 4 == 0 && oOff % 4 == 0 && oBatch % 4 == 0 && aligned16(o),
              "%s: the output view must be 16-byte aligned (ldo, oOff, oBatch multiples of 4)", fn);
  NS2_REQUIRE(ldq >= D && ldk >= D && ldv >= D, "%s: row strides must cover one head", fn);
  if (key_bias) NS2_REQUIRE(biasStart >= 0, "%s: negative biasStart", fn);
  if (k_text || v_text) {
    NS2_REQUIRE(k_text && v_text && batch == 1 && text_start >= 0 && text_start <= Lk && ld_text >= H * D,
                "%s: the text view needs k_text and v_text, batch 1, 0 <= text_start <= Lk and ld_text >= H*D", fn);
  }
  const int Lq_pad = (Lq + QPAD - 1) / QPAD * QPAD;
  const int Lk_pad = (Lk + KB - 1) / KB * KB;
  const long long bh = (long long)batch * H;
  const size_t qbytes = (size_t)bh * Lq_pad * D * sizeof(half_t);
  const size_t kbytes = (size_t)bh * Lk_pad * D * sizeof(half_t);
  const size_t bbytes = (size_t)batch * Lk_pad * sizeof(float);
  // the vectorized pack needs 16-byte aligned rows in every view it reads; then the flash
  // kernel reads Q itself and no packed Q is written
  auto al4 = [](long long x) { return x % 4 == 0; };
  const bool vec = aligned16(q) && aligned16(k) && aligned16(v) && al4(ldq) && al4(ldk) && al4(ldv) &&
                   al4(qOff) && al4(kOff) && al4(vOff) && al4(qBatch) && al4(kBatch) && al4(vBatch) &&
                   (!q_norm || aligned16(q_norm)) && (!k_norm || aligned16(k_norm)) &&
                   (!rope_cs || (aligned16(rope_cs) && al4(sin_off))) &&
                   (!k_text || (aligned16(k_text) && aligned16(v_text) && al4(ld_text)));
  if (vpk) {
    NS2_REQUIRE(!noalloc && batch == 1 && aligned16(vpk) && v_rows >= 0 && v_rows % 16 == 0 && v_rows <= Lk,
                "%s: packed values need batch 1, a 16-byte aligned buffer and 0 <= v_rows <= Lk, v_rows %% 16 == 0 "
                "(v_rows=%d Lk=%d)", fn, v_rows, Lk);
    NS2_REQUIRE(vec, "%s: packed values need 16-byte aligned views (the vectorized pack)", fn);
  }
  half_t *Qp, *Kc, *Vc;
  float* B2;
  if (noalloc) {
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t need = up(kbytes) * 2 + up(bbytes) + (vec ? 0 : up(qbytes));
    NS2_REQUIRE(need <= (size_t)NS2_NOALLOC_SCRATCH_BYTES,
                "%s: batch %d x %d heads x %d keys (D=%d) needs %zu bytes of scratch, more than the %zu "
                "of the fixed array",
                fn, batch, H, Lk, D, need, (size_t)NS2_NOALLOC_SCRATCH_BYTES);
    unsigned char* base = static_cast<unsigned char*>(ns2::noalloc_scratch());
    if (!base) return ns2::set_error(NS2_ERR_STATE, "%s: the scratch array of this device is not resolved", fn);
    Kc = reinterpret_cast<half_t*>(base);
    Vc = reinterpret_cast<half_t*>(base + up(kbytes));
    B2 = reinterpret_cast<float*>(base + 2 * up(kbytes));
    Qp = vec ? nullptr : reinterpret_cast<half_t*>(base + 2 * up(kbytes) + up(bbytes));
  } else {
    Qp = static_cast<half_t*>(ns2::workspace(1, qbytes));
    Kc = static_cast<half_t*>(ns2::workspace(2, kbytes));
    Vc = vpk ? reinterpret_cast<half_t*>(vpk) : static_cast<half_t*>(ns2::workspace(3, kbytes));
    B2 = static_cast<float*>(ns2::workspace(4, bbytes));
    if (!Qp || !Kc || !Vc || !B2) return ns2::set_error(NS2_ERR_OOM, "%s: workspace allocation failed", fn);
  }

  PackArgs pa{q, k, v, key_bias, q_norm, k_norm, rope_cs, Qp, Kc, Vc, B2,
              qOff, kOff, vOff, qBatch, kBatch, vBatch, biasBatch, sin_off,
              Lq, Lk, Lq_pad, Lk_pad, H, ldq, ldk, ldv, biasStart, rope_rows,
              scale * kLog2e, eps};
  int first_biased = Lk;  // padding keys need the mask bias too
  if (key_bias && biasStart < Lk) first_biased = biasStart;
  FlashArgs fa{Qp, Kc, Vc, B2, o, oOff, oBatch, Lq, Lk, Lq_pad, Lk_pad, H, ldo, first_biased / KB, 0, 0, 0,
               vec ? 1 : 0, q, q_norm, rope_cs, qOff, qBatch, sin_off, ldq, rope_rows, scale * kLog2e, eps};
  pa.skip_q = vec ? 1 : 0;
  pa.k2 = k_text;
  pa.v2 = v_text;
  pa.ld2 = ld_text;
  pa.kv2_start = text_start;
  pa.v_pre = vpk ? v_rows : 0;
  const bool profile = !noalloc;
  switch (D) {
    case 32: return run_attention<32>(pa, fa, batch, vec, profile);
    case 64: return run_attention<64>(pa, fa, batch, vec, profile);
    case 96: return run_attention<96>(pa, fa, batch, vec, profile);
    default: return run_attention<128>(pa, fa, batch, vec, profile);
  }
}

}  // namespace

extern "C" int ns2_attention(const float* q, const float* k, const float* v, float* o, int batch,
                             int Lq, int Lk, int H, int D, int ldq, int ldk, int ldv, int ldo,
                             long long qOff, long long kOff, long long vOff, long long oOff,
                             long long qBatch, long long kBatch, long long vBatch, long long oBatch,
                             float scale, const float* key_bias, int biasStart, long long biasBatch,
                             const float* q_norm, const float* k_norm, float eps,
                             const float* rope_cs, long long sin_off, int rope_rows) {
  return attention_call("ns2_attention", false, q, k, v, o, batch, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff,
                        vOff, oOff, qBatch, kBatch, vBatch, oBatch, scale, key_bias, biasStart, biasBatch, q_norm,
                        k_norm, eps, rope_cs, sin_off, rope_rows);
}

extern "C" int ns2_attention_text(const float* q, const float* k, const float* v, float* o, int Lq, int Lk,
                                  int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff, long long kOff,
                                  long long vOff, long long oOff, float scale, const float* key_bias,
                                  int biasStart, const float* q_norm, const float* k_norm, float eps,
                                  const float* rope_cs, long long sin_off, int rope_rows, const float* k_text,
                                  const float* v_text, int ld_text, int text_start) {
  NS2_REQUIRE(k_text && v_text, "ns2_attention_text: null k_text or v_text");
  return attention_call("ns2_attention_text", false, q, k, v, o, 1, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff,
                        vOff, oOff, 0, 0, 0, 0, scale, key_bias, biasStart, 0, q_norm, k_norm, eps, rope_cs,
                        sin_off, rope_rows, k_text, v_text, ld_text, text_start);
}

extern "C" int ns2_attention_vpacked(const float* q, const float* k, const float* v, float* o, int Lq, int Lk,
                                     int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff,
                                     long long kOff, long long vOff, long long oOff, float scale,
                                     const float* key_bias, int biasStart, const float* q_norm,
                                     const float* k_norm, float eps, const float* rope_cs, long long sin_off,
                                     int rope_rows, const float* k_text, const float* v_text, int ld_text,
                                     int text_start, uint16_t* vpk, int v_rows) {
  NS2_REQUIRE(vpk, "ns2_attention_vpacked: null vpk");
  NS2_REQUIRE(!k_text == !v_text, "ns2_attention_vpacked: k_text and v_text go together");
  return attention_call("ns2_attention_vpacked", false, q, k, v, o, 1, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff, kOff,
                        vOff, oOff, 0, 0, 0, 0, scale, key_bias, biasStart, 0, q_norm, k_norm, eps, rope_cs,
                        sin_off, rope_rows, k_text, v_text, ld_text, text_start, vpk, v_rows);
}

extern "C" size_t ns2_attention_vpack_bytes(int Lk, int H, int D) {
  if (Lk <= 0 || H <= 0 || D <= 0) return 0;
  return (size_t)H * ((Lk + KB - 1) / KB * KB) * D * sizeof(half_t);
}

extern "C" int ns2_attention_noalloc(const float* q, const float* k, const float* v, float* o, int batch,
                                     int Lq, int Lk, int H, int D, int ldq, int ldk, int ldv, int ldo,
                                     long long qOff, long long kOff, long long vOff, long long oOff,
                                     long long qBatch, long long kBatch, long long vBatch, long long oBatch,
                                     float scale, const float* key_bias, int biasStart, long long biasBatch,
                                     const float* q_norm, const float* k_norm, float eps,
                                     const float* rope_cs, long long sin_off, int rope_rows) {
  return attention_call("ns2_attention_noalloc", true, q, k, v, o, batch, Lq, Lk, H, D, ldq, ldk, ldv, ldo, qOff,
                        kOff, vOff, oOff, qBatch, kBatch, vBatch, oBatch, scale, key_bias, biasStart, biasBatch,
                        q_norm, k_norm, eps, rope_cs, sin_off, rope_rows);
}
