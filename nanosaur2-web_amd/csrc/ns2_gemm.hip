// Linear layers: C = epilogue(alpha * A W^T) with int8 ConvRot or bf16 weights.
//
// Large M runs on MFMA (v_mfma_f32_32x32x16_f16): both operands are fp16 in LDS, fp32
// accumulation. int8 weights are exact in fp16 and are decoded from bytes in the tile
// loader (bias trick: 0x6400 | (b ^ 0x80) is the half 1024 + b + 128); bf16 weights are
// converted through fp32. Activations arrive either as the rotated fp16 operand written
// by the producing row kernel (int8 layers) or as fp32 (bf16 layers), converted in the
// loader. The per-row int8 scale is applied in the epilogue, in the reference's order
// (app/gpu/gemm.js:159-164). Small M (GEMV-like, e.g. the adaLN projections of one
// conditioning vector) runs on a fp32-FMA kernel that streams the weights once.
#include "ns2_common.h"

using namespace ns2dev;

namespace {

struct GemmArgs {
  const void* A;
  const void* W;
  const float* scale;
  const float* bias;
  const float* add;
  float* C;
  const float* gate;
  long long cOff;
  long long gOff;
  int lda, ldc;
  int M, N, K;
  float alpha;
  int act, resid;
  // split-K: block z sums k tiles [z * ksteps, (z + 1) * ksteps) into part[z] ([M, N], no
  // epilogue); splitk_reduce_kernel adds the splits in z order and applies the epilogue
  float* part;
  int ksteps;
  // LoRA side path (lora_tile / lora_dot, added after the bias): lt fp32 [M][lr], lb fp16 [N][lr]; lr = 0 without
  const float* lt;
  const half_t* lb;
  int lr;
};

constexpr int BK = 64;        // k per LDS tile
constexpr int LDS_PAD = 8;    // halfs of padding per LDS row (bank spread)
constexpr int LROW = BK + LDS_PAD;

// Epilogue of one output element (gemm.js:159-164).
__device__ __forceinline__ void epilogue_store(const GemmArgs& p, int m, int n, float acc,
                                               float rs, float bi, float gt, float lora = 0.f) {
  float r = acc * p.alpha;
  r *= rs;
  r += bi;
  r += lora;  // the LoRA term, where the reference adds its delta (gemm.js:162)
  if (p.add) r += p.add[(long long)m * p.N + n];
  r = apply_act(r, p.act);
  float* c = p.C + p.cOff + (long long)m * p.ldc + n;
  if (!p.resid) *c = r;
  else if (!p.gate) *c = *c + r;
  else *c = *c + gt * r;
}

// 4 signed bytes -> 4 halfs (exact): half(0x6400 | u) = 1024 + u with u = b + 128.
__device__ __forceinline__ uint2 i8x4_to_h4(uint32_t w) {
  const uint32_t x = w ^ 0x80808080u;
  const uint32_t lo = (x & 0xffu) | ((x & 0xff00u) << 8) | 0x64006400u;
  const uint32_t hi = ((x >> 16) & 0xffu) | ((x >> 8) & 0xff0000u) | 0x64006400u;
  const half2_t off = {(half_t)1152.0f, (half_t)1152.0f};
  half2_t l = __builtin_bit_cast(half2_t, lo) - off;
  half2_t h = __builtin_bit_cast(half2_t, hi) - off;
  return make_uint2(__builtin_bit_cast(uint32_t, l), __builtin_bit_cast(uint32_t, h));
}

__device__ __forceinline__ uint32_t bf16x2_to_h2(uint32_t w) {
  const float a = __builtin_bit_cast(float, w << 16);
  const float b = __builtin_bit_cast(float, w & 0xffff0000u);
  return pack_half2(a, b);
}

// Tile loaders: global -> registers (prefetch) -> LDS (fp16, [rows][LROW]).
template <int ROWS, int NT, bool A_F32>
struct ALoader {
  // fp16 operand: 16-byte chunks of 8 k; fp32 operand: 16-byte chunks of 4 k
  static constexpr int KPC = A_F32 ? 4 : 8;
  static constexpr int CPR = BK / KPC;
  static constexpr int CHUNKS = ROWS * CPR / NT;
  static_assert(ROWS * CPR % NT == 0, "A tile not divisible");
  uint4 r[CHUNKS];
  __device__ __forceinline__ void load(const GemmArgs& p, int row0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, kc = (c % CPR) * KPC;
      const int m = row0 + row, k = k0 + kc;
      // unconditional loads from clamped addresses (a load behind a branch costs a wait each),
      // chunks outside the matrix zeroed afterwards
      const bool in = m < p.M && k < p.K;
      const long long off = (long long)(m < p.M ? m : p.M - 1) * p.lda + (k < p.K ? k : 0);
      if (A_F32)
        r[i] = *reinterpret_cast<const uint4*>(static_cast<const float*>(p.A) + off);
      else
        r[i] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.A) + off);
      const uint32_t keep = 0u - (uint32_t)in;  // mask, not a branch: a branch would wait for the load
      r[i].x &= keep; r[i].y &= keep; r[i].z &= keep; r[i].w &= keep;
    }
  }
  __device__ __forceinline__ void store(half_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, kc = (c % CPR) * KPC;
      half_t* dst = lds + row * LROW + kc;
      if (A_F32) {
        uint2 h;
        h.x = pack_half2(__builtin_bit_cast(float, r[i].x), __builtin_bit_cast(float, r[i].y));
        h.y = pack_half2(__builtin_bit_cast(float, r[i].z), __builtin_bit_cast(float, r[i].w));
        *reinterpret_cast<uint2*>(dst) = h;
      } else {
        *reinterpret_cast<uint4*>(dst) = r[i];
      }
    }
  }
};

template <int ROWS, int NT, bool W_BF16>
struct WLoader {
  // int8: 16-byte chunks of 16 k; bf16: 16-byte chunks of 8 k
  static constexpr int KPC = W_BF16 ? 8 : 16;
  static constexpr int CPR = BK / KPC;
  static constexpr int CHUNKS = ROWS * CPR / NT;
  static_assert(ROWS * CPR % NT == 0, "W tile not divisible");
  uint4 r[CHUNKS];
  __device__ __forceinline__ void load(const GemmArgs& p, int row0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, kc = (c % CPR) * KPC;
      const int n = row0 + row, k = k0 + kc;
      const bool in = n < p.N && k < p.K;
      const long long off = (long long)(n < p.N ? n : p.N - 1) * p.K + (k < p.K ? k : 0);
      if (W_BF16)
        r[i] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.W) + off);
      else
        r[i] = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(p.W) + off);
      const uint32_t keep = 0u - (uint32_t)in;  // mask, not a branch: a branch would wait for the load
      r[i].x &= keep; r[i].y &= keep; r[i].z &= keep; r[i].w &= keep;
    }
  }
  __device__ __forceinline__ void store(half_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, kc = (c % CPR) * KPC;
      half_t* dst = lds + row * LROW + kc;
      if (W_BF16) {
        uint4 h;
        h.x = bf16x2_to_h2(r[i].x);
        h.y = bf16x2_to_h2(r[i].y);
        h.z = bf16x2_to_h2(r[i].z);
        h.w = bf16x2_to_h2(r[i].w);
        *reinterpret_cast<uint4*>(dst) = h;
      } else {
        const uint2 a = i8x4_to_h4(r[i].x), b = i8x4_to_h4(r[i].y);
        const uint2 c2 = i8x4_to_h4(r[i].z), d = i8x4_to_h4(r[i].w);
        *reinterpret_cast<uint4*>(dst) = make_uint4(a.x, a.y, b.x, b.y);
        *reinterpret_cast<uint4*>(dst + 8) = make_uint4(c2.x, c2.y, d.x, d.y);
      }
    }
  }
};

// Block tile BM x BN, wave tile WM x WN of 32x32 MFMA tiles, BK = 64 per LDS stage,
// double-buffered LDS with register prefetch of the next stage.
// MFMA 32x32x16 operand layout: lane l supplies row (l % 32) of A and column (l % 32) of B,
// each with 8 consecutive k of the 16 (k = 8 * (l / 32) + e); accumulator element r of lane
// l is C[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32].
template <int BM, int BN, int WM, int WN, bool A_F32, bool W_BF16, bool LORA>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_mfma_kernel(GemmArgs p) {
  constexpr int WAVES_N = BN / WN;
  constexpr int NT = (BM / WM) * WAVES_N * 64;
  constexpr int TM = WM / 32, TN = WN / 32;
  __shared__ __attribute__((aligned(16))) half_t lds_a[2][BM * LROW];
  __shared__ __attribute__((aligned(16))) half_t lds_b[2][BN * LROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  ALoader<BM, NT, A_F32> la;
  WLoader<BN, NT, W_BF16> lw;

  float16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  int kt0 = 0, nk = (p.K + BK - 1) / BK;
  if (p.part) {
    kt0 = blockIdx.z * p.ksteps;
    nk = nk - kt0 < p.ksteps ? nk - kt0 : p.ksteps;
  }
  la.load(p, m0, kt0 * BK, tid);
  lw.load(p, n0, kt0 * BK, tid);
  const int lrow = lane & 31, lk = (lane >> 5) * 8;
  la.store(lds_a[0], tid);
  lw.store(lds_b[0], tid);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      la.load(p, m0, (kt0 + kt + 1) * BK, tid);
      lw.load(p, n0, (kt0 + kt + 1) * BK, tid);
    }
    const half_t* A = lds_a[cur] + (wm * WM + lrow) * LROW + lk;
    const half_t* B = lds_b[cur] + (wn * WN + lrow) * LROW + lk;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      half8_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const half8_t*>(A + i * 32 * LROW + ks * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *reinterpret_cast<const half8_t*>(B + j * 32 * LROW + ks * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      la.store(lds_a[cur ^ 1], tid);
      lw.store(lds_b[cur ^ 1], tid);
    }
    __syncthreads();
  }

  // (the launcher splits K only on grids of 64x64 tiles)
  if constexpr (BM * BN <= 64 * 64) if (p.part) {
    float* part = p.part + (long long)blockIdx.z * p.M * p.N;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * WN + j * 32 + lrow;
      if (n >= p.N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (m < p.M) part[(long long)m * p.N + n] = acc[i][j][r];
        }
    }
    return;
  }

  // epilogue
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn * WN + j * 32 + lrow;
    if (n >= p.N) continue;
    const float rs = p.scale ? p.scale[n] : 1.0f;
    const float bi = p.bias ? p.bias[n] : 0.0f;
    const float gt = p.gate ? p.gate[p.gOff + n] : 1.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float16_t d;
      if constexpr (LORA) {
        const int ml = m0 + wm * WM + i * 32 + lrow;
        d = lora_tile(p.lt, p.lb, p.lr, ml < p.M ? ml : p.M - 1, n, lane >> 5);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < p.M) epilogue_store(p, m, n, acc[i][j][r], rs, bi, gt, LORA ? d[r] : 0.f);
      }
    }
  }
}

// Split-K reduction: the splits summed in z order (deterministic), then the GEMM epilogue.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs p, int splits) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long mn = (long long)p.M * p.N;
  if (i >= mn) return;
  float acc = 0.f;
  for (int z = 0; z < splits; ++z) acc += p.part[z * mn + i];
  const int m = (int)(i / p.N), n = (int)(i % p.N);
  epilogue_store(p, m, n, acc, p.scale ? p.scale[n] : 1.0f, p.bias ? p.bias[n] : 0.0f,
                 p.gate ? p.gate[p.gOff + n] : 1.0f, p.lr ? lora_dot(p.lt, p.lb, p.lr, m, n) : 0.f);
}

// Split-K sum of one output row followed by the Gemma3 sublayer norms of that row (one block
// per row): t = epilogue(sum of the splits), x += rmsnorm(t) * w_add, y = rmsnorm(x) * w_out
// (y optional). Thread i owns columns i + 256 j (j < C, C = ceil(N / 256)); the loads of 16
// splits go out together (one round trip for the 16 down-projection shares of the encoder's MLP)
// from clamped addresses, and the splits are added in split order, as splitk_reduce_kernel adds
// them.
constexpr int kRowNormCols = 4;
constexpr int kRowNormSplitsInFlight = 16;
constexpr int kRowNormMaxN = 256 * kRowNormCols;
struct RowNorm {
  float* x;
  const float* w_add;
  const float* w_out;
  float* y;
  float eps;
  // y as the tiled fp16 operand of the next linear (K = N columns) instead of fp32: each value
  // rounded once to nearest
  uint16_t* yt;
};
template <int C>
__global__ __launch_bounds__(256) void splitk_add_rmsnorm_kernel(GemmArgs p, int splits, RowNorm rn) {
  constexpr int ZB = kRowNormSplitsInFlight;
  __shared__ float red[4];
  const int N = p.N, tid = threadIdx.x;
  const long long mn = (long long)p.M * N, row = (long long)blockIdx.x * N;
  int col[C];
  float acc[C], xv[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int n = tid + 256 * j;
    col[j] = n < N ? n : N - 1;
    acc[j] = 0.f;
    xv[j] = rn.x[row + col[j]];
  }
  for (int z0 = 0; z0 < splits; z0 += ZB) {
    float v[ZB][C];
#pragma unroll
    for (int k = 0; k < ZB; ++k) {
      const long long zo = (long long)(z0 + k < splits ? z0 + k : splits - 1) * mn + row;
#pragma unroll
      for (int j = 0; j < C; ++j) v[k][j] = p.part[zo + col[j]];
    }
#pragma unroll
    for (int k = 0; k < ZB; ++k)
#pragma unroll
      for (int j = 0; j < C; ++j)
        if (z0 + k < splits) acc[j] += v[k][j];
  }
  float t[C], ss = 0.f;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int n = col[j];
    float r = acc[j] * p.alpha;
    if (p.scale) r *= p.scale[n];
    if (p.bias) r += p.bias[n];
    t[j] = r;
    if (tid + 256 * j < N) ss += r * r;
  }
  const float r1 = rsqrtf(block_sum(ss, red) / (float)N + rn.eps);
  float sx = 0.f;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const float v = xv[j] + t[j] * r1 * rn.w_add[col[j]];
    t[j] = v;
    if (tid + 256 * j < N) {
      rn.x[row + col[j]] = v;
      sx += v * v;
    }
  }
  if (!rn.y && !rn.yt) return;
  const float r2 = rsqrtf(block_sum(sx, red) / (float)N + rn.eps);
#pragma unroll
  for (int j = 0; j < C; ++j)
    if (tid + 256 * j < N) {
      float v = t[j] * r2 * rn.w_out[col[j]];
      if (rn.yt) {
        asm volatile("" : "+v"(v));  // the fp32 value, then one rounding (no fused conversion)
        reinterpret_cast<half_t*>(rn.yt)[tiled_off(blockIdx.x, col[j], N)] = (half_t)v;
      } else {
        rn.y[row + col[j]] = v;
      }
    }
}

// The row kernel with as many column slots per thread as N needs (N <= kRowNormMaxN).
void launch_add_rmsnorm(const GemmArgs& p, int splits, const RowNorm& rn, hipStream_t s) {
  if (p.N <= 512) splitk_add_rmsnorm_kernel<2><<<p.M, 256, 0, s>>>(p, splits, rn);
  else if (p.N <= 768) splitk_add_rmsnorm_kernel<3><<<p.M, 256, 0, s>>>(p, splits, rn);
  else splitk_add_rmsnorm_kernel<kRowNormCols><<<p.M, 256, 0, s>>>(p, splits, rn);
}

// Split-K sum of a stacked q|k|v product followed by the per-head norms of app/gpu/ops.js:
// 133-138 on its q and k heads (Gemma3, app/models/gemma3.js:64-67): one block of D threads per
// row, thread i owning dim i of every head. Heads h < H1 are RMS-normed with w1, heads
// [H1, H1 + H2) with w2, then split-half RoPE on rows < rope_rows (pair i, i + D/2; cos at
// cs[row*D/2 + i], sin at cs[sin_off + row*D/2 + i]); the remaining heads (the values) are stored
// as summed. The splits are added in split order, as splitk_reduce_kernel adds them.
// With kv16 set, heads h >= H1 (the keys and values) are stored as fp16 at
// kv16[row*ldkv + (h - H1)*D + i] instead of fp32 in C: the fp32 value rounded once to nearest.
struct HeadNorm {
  const float* w1;
  int H1;
  const float* w2;
  int H2, D;
  const float* cs;
  long long sin_off;
  int rope_rows;
  float eps;
  half_t* kv16;
  long long ldkv;
};
constexpr int kHeadNormMaxHeads = 8;
template <int D>
__global__ __launch_bounds__(D) void splitk_head_norm_kernel(GemmArgs p, int splits, HeadNorm hn) {
  constexpr int MH = kHeadNormMaxHeads;
  __shared__ float red[D / 64 * MH];
  __shared__ float row_buf[MH * D];
  const int tid = threadIdx.x, heads = p.N / D;
  const long long mn = (long long)p.M * p.N, m = blockIdx.x;
  // every load of the row first (unconditional, from clamped addresses): the split partials
  // of all heads, the norm weights and the rotation's cos / sin
  const float* part = p.part + m * p.N + tid;
  float acc[MH];
#pragma unroll
  for (int h = 0; h < MH; ++h) acc[h] = 0.f;
  for (int z = 0; z < splits; ++z) {
#pragma unroll
    for (int h = 0; h < MH; ++h) acc[h] += part[z * mn + (long long)(h < heads ? h : heads - 1) * D];
  }
  const float w1 = hn.H1 ? hn.w1[tid] : 0.f, w2 = hn.H2 ? hn.w2[tid] : 0.f;
  const int half = D / 2, i = tid % half;
  const bool rope = hn.cs && m < hn.rope_rows;  // uniform per block
  const float c = rope ? hn.cs[m * half + i] : 1.f, sn = rope ? hn.cs[hn.sin_off + m * half + i] : 0.f;
  float* out = p.C + p.cOff + m * p.ldc + tid;
  const int normed = hn.H1 + hn.H2;
  float r[MH];
#pragma unroll
  for (int h = 0; h < MH; ++h) {
    r[h] = acc[h] * p.alpha;
    if (p.scale) r[h] *= p.scale[(h < heads ? h : heads - 1) * D + tid];
    if (p.bias) r[h] += p.bias[(h < heads ? h : heads - 1) * D + tid];
  }
  // the normed heads' sums of squares together: wave sums, one barrier, then each thread adds
  // the waves' partials in wave order (block_sum's order)
  const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int h = 0; h < MH; ++h) {
    if (h >= normed) break;
    const float ws = wave_sum(r[h] * r[h]);
    if (lane == 0) red[wv * MH + h] = ws;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < MH; ++h) {
    if (h >= normed) break;
    float t = 0.f;
    for (int w = 0; w < D / 64; ++w) t += red[w * MH + h];
    r[h] = r[h] * rsqrtf(t / (float)D + hn.eps) * (h < hn.H1 ? w1 : w2);
  }
  if (rope) {
    // split-half RoPE of every normed head, the partners through LDS (one barrier)
#pragma unroll
    for (int h = 0; h < MH; ++h)
      if (h < normed) row_buf[h * D + tid] = r[h];
    __syncthreads();
#pragma unroll
    for (int h = 0; h < MH; ++h) {
      if (h >= normed) break;
      const float other = row_buf[h * D + (tid < half ? tid + half : tid - half)];
      r[h] = tid < half ? r[h] * c - other * sn : r[h] * c + other * sn;
    }
  }
#pragma unroll
  for (int h = 0; h < MH; ++h) {
    if (h >= heads) break;
    float v = r[h];
    if (hn.kv16 && h >= hn.H1) {  // uniform per block
      // the fp32 value as the fp32 store would hold it (no multiply-add fused with the conversion)
      asm volatile("" : "+v"(v));
      hn.kv16[m * hn.ldkv + (long long)(h - hn.H1) * D + tid] = (half_t)v;
    } else {
      out[(long long)h * D] = v;
    }
  }
}

// Split-K sum of a gate/up product followed by the GLU: y[m][i] = act(t[m][i]) * t[m][I + i]
// with t = epilogue(sum of the splits), N = 2I (gate rows first, as concatLinears stacks them).
// The splits are added in split order, as splitk_reduce_kernel adds them.
__global__ __launch_bounds__(256) void splitk_glu_kernel(GemmArgs p, int splits, float* __restrict__ y, int glu_act) {
  const int I = p.N / 2;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)p.M * I) return;
  const long long m = i / I, j = i % I;
  const long long mn = (long long)p.M * p.N, g0 = m * p.N + j;
  float g = 0.f, u = 0.f;
  for (int z = 0; z < splits; ++z) {
    g += p.part[z * mn + g0];
    u += p.part[z * mn + g0 + I];
  }
  g *= p.alpha;
  u *= p.alpha;
  if (p.scale) {
    g *= p.scale[j];
    u *= p.scale[j + I];
  }
  if (p.bias) {
    g += p.bias[j];
    u += p.bias[j + I];
  }
  y[i] = apply_act(g, glu_act) * u;
}

// Split-K sum of a gate/up product, its GLU, and the linear after it split over the GLU
// output's GS-column groups (Gemma3's MLP, app/models/gemma3.js:79-83). Block (16 rows, group r)
// forms y = act(gate) * up for its rows and the group's columns with splitk_glu_kernel's
// arithmetic, rounds y to fp16 into LDS (as the next linear's loader rounds its input) and
// multiplies it by the next weight's GS columns of group r (fp16 tiles, tile_w16_kernel's
// layout) on v_mfma_f32_16x16x16_f16: share r of that product, out[r][m][n] fp32 for n < Nd.
// The I/GS shares, summed in r order, are the product without bias. Each wave takes 16-column
// tiles n0 = 16w, 16(w + 8), ...; the weight fragments of its first JC tiles are loaded before
// the split sums are read (they do not depend on them), the rest JC tiles per round trip.
// GLU output columns per share: 128 makes 16 x 16 = 256 (16 rows, group) units at 256 rows, each
// streaming 160 KB of the down weight from L2 (256: 128 units of 320 KB, 11.3 us per layer
// before the column ranges below)
constexpr int kGluDownGroup = 128;
struct GluDown {
  const half_t* wd;  // the next weight [Nd][I] as fp16 tiles
  float* out;        // [I/GS][M][Nd]
  int Nd, act;
  // blocks per (16 rows, group), blockIdx.z, each a range of the Nd/16 column tiles (each repeats
  // the group's GLU): at 256 rows two blocks per CU, each streaming half the group's weight slice
  int ncs;
};
// Column ranges per (16 rows, group): doubled while the grid stays within two blocks per CU
// and every block keeps at least 8 of the 16-column tiles (one per wave).
constexpr long long kGluDownMaxBlocks = 2 * 256;
inline int glu_down_ranges(int M, int N, int Nd) {
  const long long blocks = (long long)((M + 15) / 16) * (N / 2 / kGluDownGroup);
  int ncs = 1;
  while (ncs < 4 && blocks * ncs * 2 <= kGluDownMaxBlocks && Nd / 16 >= ncs * 2 * 8) ncs *= 2;
  return ncs;
}
template <int GS>
__global__ __launch_bounds__(512) void splitk_glu_down_kernel(GemmArgs p, int splits, GluDown gd) {
  constexpr int NW = 8, OS = GS + 8, DB = GS / 16, JC = 5, CPT = GS * 16 / 512;  // GLU columns per thread
  __shared__ __attribute__((aligned(16))) half_t g16[16 * OS];
  const int I = p.N / 2;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
  const int m0 = blockIdx.x * 16, j0 = blockIdx.y * GS, nt = gd.Nd / 16;
  const int jlo = (int)blockIdx.z * nt / gd.ncs, jhi = ((int)blockIdx.z + 1) * nt / gd.ncs;
  // lane's fragment t of column tile jt: tiled_off(16 jt + col, j0 + 16 t + 4 grp, I), which is
  // the offset for t = 0 plus 1024 t (j0 and 16 t + 4 grp stay inside one 64-column k-tile
  // pair of chunks: k >> 6 = j0/64 + t/4, chunk 2 (t % 4) + grp/2, element 4 (grp & 1))
  half4_t bf[JC][DB];
  auto load_w = [&](int jt0) {
#pragma unroll
    for (int c = 0; c < JC; ++c) {
      const int jt = jt0 + c * NW;
      if (jt < jhi) {  // uniform per wave
        const half_t* wrow = gd.wd + tiled_off(16 * jt + col, j0 + 4 * grp, I);
#pragma unroll
        for (int t = 0; t < DB; ++t) bf[c][t] = *reinterpret_cast<const half4_t*>(wrow + 1024 * t);
      }
    }
  };
  load_w(jlo + wave);
  {
    // thread: row rr, columns c8 .. c8 + CPT - 1 of the group (rows past M repeat the last row)
    static_assert(CPT == 4 || CPT == 8, "4 or 8 GLU columns per thread");
    const int rr = tid / (GS / CPT), c8 = (tid % (GS / CPT)) * CPT;
    const long long m = m0 + rr < p.M ? m0 + rr : p.M - 1;
    const long long mn = (long long)p.M * p.N;
    const float* gp = p.part + m * p.N + j0 + c8;
    float g[CPT], u[CPT];
#pragma unroll
    for (int e = 0; e < CPT; ++e) g[e] = u[e] = 0.f;
    // two splits' loads in flight at a time (the weight fragments above hold most registers)
#pragma unroll 2
    for (int z = 0; z < splits; ++z) {
#pragma unroll
      for (int e4 = 0; e4 < CPT; e4 += 4) {
        const float4 gv = *reinterpret_cast<const float4*>(gp + z * mn + e4);
        const float4 uv = *reinterpret_cast<const float4*>(gp + z * mn + I + e4);
        g[e4] += gv.x, g[e4 + 1] += gv.y, g[e4 + 2] += gv.z, g[e4 + 3] += gv.w;
        u[e4] += uv.x, u[e4 + 1] += uv.y, u[e4 + 2] += uv.z, u[e4 + 3] += uv.w;
      }
    }
    half_t hv[CPT];
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
      const int j = j0 + c8 + e;
      float a = g[e] * p.alpha, b = u[e] * p.alpha;
      if (p.scale) {
        a *= p.scale[j];
        b *= p.scale[j + I];
      }
      if (p.bias) {
        a += p.bias[j];
        b += p.bias[j + I];
      }
      float y = apply_act(a, gd.act) * b;
      // the fp32 value first, as the GLU kernel stores it: no multiply fused into the conversion
      asm volatile("" : "+v"(y));
      hv[e] = (half_t)y;
    }
    if constexpr (CPT == 8) {
      *reinterpret_cast<half8_t*>(&g16[rr * OS + c8]) = half8_t{hv[0], hv[1], hv[2], hv[3], hv[4], hv[5], hv[6], hv[7]};
    } else {
      *reinterpret_cast<half4_t*>(&g16[rr * OS + c8]) = half4_t{hv[0], hv[1], hv[2], hv[3]};
    }
  }
  __syncthreads();
  half4_t af[DB];
#pragma unroll
  for (int t = 0; t < DB; ++t) af[t] = *reinterpret_cast<const half4_t*>(&g16[col * OS + 16 * t + 4 * grp]);
  for (int jt0 = jlo + wave; jt0 < jhi; jt0 += JC * NW) {
    if (jt0 != jlo + wave) load_w(jt0);
#pragma unroll
    for (int c = 0; c < JC; ++c) {
      const int jt = jt0 + c * NW;
      if (jt < jhi) {
        float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < DB; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x16f16(af[t], bf[c][t], acc, 0, 0, 0);
        // acc[i]: row m0 + 4 grp + i, column 16 jt + col
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + 4 * grp + i;
          if (m < p.M) gd.out[((long long)blockIdx.y * p.M + m) * gd.Nd + 16 * jt + col] = acc[i];
        }
      }
    }
  }
}

// Small-M path: one wave per output column n, all M (<= MR <= 8) rows, fp32 FMA.
// A: fp32 [M, lda] (bf16 layers) or rotated fp16 [M, lda] (int8 layers).
template <bool W_BF16, int MR>
__global__ __launch_bounds__(256) void gemv_kernel(GemmArgs p) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= p.N) return;
  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
  for (int k = lane * 8; k < p.K; k += 512) {
    // every load of the step is issued before the first use: W's 8 values and the MR rows of A
    // (rows past M repeat the last row, so the loads are unconditional; their sums are not stored)
    uint4 wq;
    uint4 ar[MR][2];
    if (W_BF16) {
      wq = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.W) + (long long)n * p.K + k);
    } else {
      const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(p.W) + (long long)n * p.K + k);
      wq = make_uint4(q.x, q.y, 0u, 0u);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const int mr = m < p.M ? m : p.M - 1;
      if (W_BF16) {
        const float* ap = static_cast<const float*>(p.A) + (long long)mr * p.lda + k;
        ar[m][0] = *reinterpret_cast<const uint4*>(ap);
        ar[m][1] = *reinterpret_cast<const uint4*>(ap + 4);
      } else {
        ar[m][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.A) + (long long)mr * p.lda + k);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    float w[8];
    if (W_BF16) {
      const uint32_t qq[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w[2 * j] = __builtin_bit_cast(float, qq[j] << 16);
        w[2 * j + 1] = __builtin_bit_cast(float, qq[j] & 0xffff0000u);
      }
    } else {
      const uint32_t qq[2] = {wq.x, wq.y};
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = (float)(int8_t)((qq[j >> 2] >> (8 * (j & 3))) & 0xff);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float a[8];
      if (W_BF16) {
        const float4 x0 = __builtin_bit_cast(float4, ar[m][0]);
        const float4 x1 = __builtin_bit_cast(float4, ar[m][1]);
        a[0] = x0.x; a[1] = x0.y; a[2] = x0.z; a[3] = x0.w;
        a[4] = x1.x; a[5] = x1.y; a[6] = x1.z; a[7] = x1.w;
      } else {
        const half8_t h = __builtin_bit_cast(half8_t, ar[m][0]);
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = (float)h[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[m] = fmaf(a[j], w[j], acc[m]);
    }
  }
  const float rs = p.scale ? p.scale[n] : 1.0f;
  const float bi = p.bias ? p.bias[n] : 0.0f;
  const float gt = p.gate ? p.gate[p.gOff + n] : 1.0f;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m < p.M) {
      const float s = wave_sum(acc[m]);
      // LoRA term: the lanes split the rank
      float d = 0.f;
      if (p.lr) {
        for (int k = lane; k < p.lr; k += 64) d += p.lt[(long long)m * p.lr + k] * (float)p.lb[(long long)n * p.lr + k];
        d = wave_sum(d);
      }
      if (lane == 0) epilogue_store(p, m, n, s, rs, bi, gt, d);
    }
  }
}

// One-row bf16 GEMV (the adaLN and embedder projections of one conditioning vector) for
// K = 512 KS: every wave owns CPW output columns and issues the loads of all its weight rows
// (CPW x KS 16-byte chunks per lane) and of the input row before any arithmetic, so a wave keeps
// CPW * K * 2 bytes in flight and the grid has CPW times fewer, longer-lived waves than one
// wave per column. Sums over k in the order of gemv_kernel's lanes and steps.
template <int CPW, int KS>
__global__ __launch_bounds__(256) void gemv1_bf16_kernel(GemmArgs p) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * CPW;
  if (n0 >= p.N) return;
  uint4 wq[CPW][KS];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int n = n0 + c < p.N ? n0 + c : p.N - 1;  // clamped: unconditional loads
#pragma unroll
    for (int s = 0; s < KS; ++s)
      wq[c][s] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.W) + (long long)n * p.K + s * 512 + lane * 8);
  }
  float4 ar[KS][2];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const float* ap = static_cast<const float*>(p.A) + s * 512 + lane * 8;
    ar[s][0] = *reinterpret_cast<const float4*>(ap);
    ar[s][1] = *reinterpret_cast<const float4*>(ap + 4);
  }
  __builtin_amdgcn_sched_barrier(0);
  float acc[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    acc[c] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t qq[4] = {wq[c][s].x, wq[c][s].y, wq[c][s].z, wq[c][s].w};
      const float a[8] = {ar[s][0].x, ar[s][0].y, ar[s][0].z, ar[s][0].w, ar[s][1].x, ar[s][1].y, ar[s][1].z, ar[s][1].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[c] = fmaf(a[2 * j], __builtin_bit_cast(float, qq[j] << 16), acc[c]);
        acc[c] = fmaf(a[2 * j + 1], __builtin_bit_cast(float, qq[j] & 0xffff0000u), acc[c]);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int n = n0 + c;
    const float sum = wave_sum(acc[c]);
    float d = 0.f;
    if (p.lr) {
      for (int k = lane; k < p.lr; k += 64) d += p.lt[k] * (float)p.lb[(long long)(n < p.N ? n : p.N - 1) * p.lr + k];
      d = wave_sum(d);
    }
    if (lane == 0 && n < p.N) {
      const float bi = p.bias ? p.bias[n] : 0.0f;
      const float gt = p.gate ? p.gate[p.gOff + n] : 1.0f;
      epilogue_store(p, 0, n, sum, 1.0f, bi, gt, d);
    }
  }
}

// fp32 [rows, lda] (already rotated) -> fp16 [rows, cols]
__global__ __launch_bounds__(256) void cast_f16_kernel(const float* __restrict__ x, int ldx,
                                                        uint16_t* __restrict__ y, int rows,
                                                        int cols) {
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= (long long)rows * cols) return;
  const long long r = i / cols, c = i % cols;
  const float4 v = *reinterpret_cast<const float4*>(x + r * ldx + c);
  uint2 o;
  o.x = pack_half2(v.x, v.y);
  o.y = pack_half2(v.z, v.w);
  *reinterpret_cast<uint2*>(y + i) = o;
}

// ---- LoRA down-projection -------------------------------------------------------------------
// t[M][R] = x A^T for the LoRA side path (A fp16 [R][K], the stacked down-projections). A block
// of NWV waves takes 32 rows; wave w takes the k-steps w, w + NWV, ... of 16, and the partial
// 32 x R accumulators are summed through LDS. RT = R / 32 output tiles of 32 columns.
template <int RT>
constexpr int lora_waves() { return RT <= 4 ? 8 : 4; }

template <int XFMT, int RT>
__global__ __launch_bounds__(64 * lora_waves<RT>()) void lora_down_kernel(const void* __restrict__ x, int ldx,
                                                                          const half_t* __restrict__ A,
                                                                          float* __restrict__ t, int M, int K) {
  constexpr int R = 32 * RT;
  constexpr int kLoraWaves = lora_waves<RT>();
  __shared__ float red[kLoraWaves - 1][RT][16][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lq = lane & 31, hi = lane >> 5;
  const int m0 = blockIdx.x * 32;
  const int m = m0 + lq < M ? m0 + lq : M - 1;  // rows past M read the last row (not stored)
  float16_t acc[RT];
#pragma unroll
  for (int j = 0; j < RT; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  // k-steps of 16 (k = 16 s + 8 hi), s = wave + kLoraWaves * j; batches of NB steps issue all
  // their loads (from clamped addresses; steps past K are zeroed) before their products
  constexpr int NB = RT <= 2 ? 6 : (RT <= 4 ? 3 : 2);
  const int steps = K / 16;
  const int mine = steps > wave ? (steps - wave + kLoraWaves - 1) / kLoraWaves : 0;
  for (int j0 = 0; j0 < mine; j0 += NB) {
    half8_t a[NB], b[NB][RT];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int sidx = wave + kLoraWaves * (j0 + u);
      const int k = (sidx < steps ? sidx : steps - 1) * 16 + 8 * hi;
      if constexpr (XFMT == 0) {
        const float* xp = static_cast<const float*>(x) + (long long)m * ldx + k;
        const float4 u0 = *reinterpret_cast<const float4*>(xp);
        const float4 u1 = *reinterpret_cast<const float4*>(xp + 4);
        a[u] = half8_t{(half_t)u0.x, (half_t)u0.y, (half_t)u0.z, (half_t)u0.w,
                       (half_t)u1.x, (half_t)u1.y, (half_t)u1.z, (half_t)u1.w};
      } else if constexpr (XFMT == 1) {
        a[u] = *reinterpret_cast<const half8_t*>(static_cast<const half_t*>(x) + (long long)m * ldx + k);
      } else {
        a[u] = *reinterpret_cast<const half8_t*>(static_cast<const half_t*>(x) + tiled_off(m, k, K));
      }
#pragma unroll
      for (int j = 0; j < RT; ++j) b[u][j] = *reinterpret_cast<const half8_t*>(A + (long long)(32 * j + lq) * K + k);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (j0 + u >= mine) a[u] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < RT; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[u], b[u][j], acc[j], 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[wave - 1][j][r][lane] = acc[j][r];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int j = 0; j < RT; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = acc[j][r];
#pragma unroll
      for (int w = 0; w < kLoraWaves - 1; ++w) v += red[w][j][r][lane];
      const int row = m0 + 8 * (r >> 2) + 4 * hi + (r & 3);
      if (row < M) t[(long long)row * R + 32 * j + lq] = v;
    }
}

// The same on v_mfma_f32_16x16x32_f16 for K % 32 == 0: a block of 8 waves takes 16 rows and
// 32 columns of t (blockIdx.y: columns 32y .. 32y+31 of R), so the 3952 image rows make 247
// blocks at rank 32 and the 256 text rows 128 blocks at rank 256 (the 32-row kernel left CUs
// idle: 10.6 us per call at rank 32, 46 us for 256 rows at rank 256). Lane l supplies row l%16
// of x and of A with k = 32s + 8(l/16) .. +7; the accumulator element i of lane l is
// t[4(l/16) + i][32y + 16j + l%16]. Every load of a wave's k-steps is issued before its products.
template <int XFMT>
__global__ __launch_bounds__(512) void lora_down16_kernel(const void* __restrict__ x, int ldx,
                                                          const half_t* __restrict__ A, float* __restrict__ t,
                                                          int M, int K, int R) {
  constexpr int RB = 2, NWV = 8, NB = 6;
  A += (long long)blockIdx.y * 32 * K;
  t += blockIdx.y * 32;
  __shared__ float red[NWV - 1][RB][4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, kq = lane >> 4;
  const int m0 = blockIdx.x * 16;
  const int m = m0 + l16 < M ? m0 + l16 : M - 1;  // rows past M read the last row (not stored)
  float4_t acc[RB];
#pragma unroll
  for (int j = 0; j < RB; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int steps = K / 32;
  const int mine = steps > wave ? (steps - wave + NWV - 1) / NWV : 0;
  for (int j0 = 0; j0 < mine; j0 += NB) {
    half8_t a[NB], b[NB][RB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int sidx = wave + NWV * (j0 + u);
      const int k = (sidx < steps ? sidx : steps - 1) * 32 + 8 * kq;
      if constexpr (XFMT == 0) {
        const float* xp = static_cast<const float*>(x) + (long long)m * ldx + k;
        const float4 u0 = *reinterpret_cast<const float4*>(xp);
        const float4 u1 = *reinterpret_cast<const float4*>(xp + 4);
        a[u] = half8_t{(half_t)u0.x, (half_t)u0.y, (half_t)u0.z, (half_t)u0.w,
                       (half_t)u1.x, (half_t)u1.y, (half_t)u1.z, (half_t)u1.w};
      } else if constexpr (XFMT == 1) {
        a[u] = *reinterpret_cast<const half8_t*>(static_cast<const half_t*>(x) + (long long)m * ldx + k);
      } else {
        a[u] = *reinterpret_cast<const half8_t*>(static_cast<const half_t*>(x) + tiled_off(m, k, K));
      }
#pragma unroll
      for (int j = 0; j < RB; ++j) b[u][j] = *reinterpret_cast<const half8_t*>(A + (long long)(16 * j + l16) * K + k);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (j0 + u >= mine) a[u] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < RB; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], b[u][j], acc[j], 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave - 1][j][i][lane] = acc[j][i];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int j = 0; j < RB; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[j][i];
#pragma unroll
      for (int w = 0; w < NWV - 1; ++w) v += red[w][j][i][lane];
      const int row = m0 + 4 * kq + i;
      if (row < M) t[(long long)row * R + 16 * j + l16] = v;
    }
}

constexpr int kGemvMaxM = 8;
constexpr long long kSmallGridBlocks = 256;  // one block per CU
constexpr int kMaxSplits = 16;
// rn: a row post-op (Gemma3's sublayer norms). It takes the 64x64 split-K path at any M, with
// the row kernel in place of the split-K reduce (a single split when K is short).
// glu_y: a GLU post-op (y [M, N/2] = act(gate) * up, act glu_act), on the same split-K path.
// hn: the per-head norms of a stacked q|k|v product (Gemma3), on the same split-K path.
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <bool A_F32, bool W_BF16>
int launch_gemm(const GemmArgs& p, const char* name, const RowNorm* rn = nullptr, float* glu_y = nullptr,
                int glu_act = 0, const HeadNorm* hn = nullptr, const GluDown* gd = nullptr) {
  hipStream_t s = ns2::stream();
  const bool post = rn || glu_y || hn || gd;
  ns2::ProfScope prof_(rn ? "gemm_bf16_add_rmsnorm" : glu_y ? "gemm_bf16_glu" : gd ? "gemm_bf16_glu_down" : hn ? "gemm_bf16_head_norm"
                          : p.M <= kGemvMaxM ? (W_BF16 ? "gemv_bf16" : "gemv_i8") : (W_BF16 ? "gemm_bf16" : "gemm_i8"));
  const long long big_tiles = (long long)((p.N + 127) / 128) * ((p.M + 127) / 128);
  if (!post && p.M == 1 && W_BF16 && A_F32 && p.K % 512 == 0 && p.K <= 2048 && aligned16(p.A)) {
    constexpr int CPW = 4;
    const dim3 grid((p.N + 4 * CPW - 1) / (4 * CPW));
    switch (p.K / 512) {
      case 1: gemv1_bf16_kernel<CPW, 1><<<grid, 256, 0, s>>>(p); break;
      case 2: gemv1_bf16_kernel<CPW, 2><<<grid, 256, 0, s>>>(p); break;
      case 3: gemv1_bf16_kernel<CPW, 3><<<grid, 256, 0, s>>>(p); break;
      default: gemv1_bf16_kernel<CPW, 4><<<grid, 256, 0, s>>>(p); break;
    }
  } else if (!post && p.M <= kGemvMaxM) {
    // row count rounded up to 1, 2, 4 or 8: no duplicate A loads for the common M = 1
    const dim3 grid((p.N + 3) / 4);
    if (p.M == 1) gemv_kernel<W_BF16, 1><<<grid, 256, 0, s>>>(p);
    else if (p.M == 2) gemv_kernel<W_BF16, 2><<<grid, 256, 0, s>>>(p);
    else if (p.M <= 4) gemv_kernel<W_BF16, 4><<<grid, 256, 0, s>>>(p);
    else gemv_kernel<W_BF16, 8><<<grid, 256, 0, s>>>(p);
  } else if (!post && big_tiles >= 2 * kSmallGridBlocks && p.K > 256) {
    // 128x128 tiles only where they make two full rounds over the CUs and K is not short: at
    // 3952 x 1536 they make 1.45 rounds and the 64x64 grid is faster (x 1536 x 1536 with +=:
    // 79.4 -> 70.3 us; x 1536 x 64: 17.7 -> 11.9 us; the same results)
    constexpr int BM = 128, BN = 128, WM = 64, WN = 64;
    dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM);
    if (p.lr) gemm_mfma_kernel<BM, BN, WM, WN, A_F32, W_BF16, true><<<grid, (BM / WM) * (BN / WN) * 64, 0, s>>>(p);
    else gemm_mfma_kernel<BM, BN, WM, WN, A_F32, W_BF16, false><<<grid, (BM / WM) * (BN / WN) * 64, 0, s>>>(p);
  } else {
    // Too few 128x128 tiles to fill 256 CUs (a short sequence): 64x64 tiles, and when even
    // those leave the chip idle, split K over blockIdx.z (at least 4 k tiles per split).
    constexpr int BM = 64, BN = 64, WM = 32, WN = 32;
    const long long tiles = (long long)((p.N + BN - 1) / BN) * ((p.M + BM - 1) / BM);
    const int nk = (p.K + BK - 1) / BK;
    int splits = (int)(2 * kSmallGridBlocks / tiles);
    if (splits > nk / 4) splits = nk / 4;
    if (splits > kMaxSplits) splits = kMaxSplits;
    if (splits < 1) splits = 1;
    GemmArgs q = p;
    if (splits > 1 || post) {
      q.ksteps = (nk + splits - 1) / splits;
      splits = (nk + q.ksteps - 1) / q.ksteps;
      q.part = static_cast<float*>(ns2::workspace(5, (size_t)splits * p.M * p.N * sizeof(float)));
      if (!q.part) return ns2::set_error(NS2_ERR_OOM, "%s: split-K workspace allocation failed", name);
    }
    dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, splits);
    if (q.lr) gemm_mfma_kernel<BM, BN, WM, WN, A_F32, W_BF16, true><<<grid, (BM / WM) * (BN / WN) * 64, 0, s>>>(q);
    else gemm_mfma_kernel<BM, BN, WM, WN, A_F32, W_BF16, false><<<grid, (BM / WM) * (BN / WN) * 64, 0, s>>>(q);
    if (rn) {
      launch_add_rmsnorm(q, splits, *rn, s);
    } else if (hn) {
      if (hn->D == 64) splitk_head_norm_kernel<64><<<p.M, 64, 0, s>>>(q, splits, *hn);
      else if (hn->D == 128) splitk_head_norm_kernel<128><<<p.M, 128, 0, s>>>(q, splits, *hn);
      else splitk_head_norm_kernel<256><<<p.M, 256, 0, s>>>(q, splits, *hn);
    } else if (gd) {
      splitk_glu_down_kernel<kGluDownGroup>
          <<<dim3((p.M + 15) / 16, p.N / 2 / kGluDownGroup, gd->ncs), 512, 0, s>>>(q, splits, *gd);
    } else if (glu_y) {
      const long long n = (long long)p.M * (p.N / 2);
      splitk_glu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(q, splits, glu_y, glu_act);
    } else if (splits > 1) {
      const long long mn = (long long)p.M * p.N;
      splitk_reduce_kernel<<<(unsigned)((mn + 255) / 256), 256, 0, s>>>(q, splits);
    }
  }
  NS2_LAUNCHED(name);
  return NS2_OK;
}

int check_common(const GemmArgs& p, const char* name) {
  NS2_REQUIRE(p.A && p.W && p.C, "%s: null A, W or C", name);
  NS2_REQUIRE(p.M >= 0 && p.N > 0 && p.K > 0, "%s: bad sizes M=%d N=%d K=%d", name, p.M, p.N, p.K);
  NS2_REQUIRE(p.K % 16 == 0, "%s: K=%d must be a multiple of 16", name, p.K);
  NS2_REQUIRE(p.lda >= p.K && p.lda % 8 == 0, "%s: lda=%d must be >= K and a multiple of 8", name, p.lda);
  NS2_REQUIRE(p.ldc >= p.N, "%s: ldc=%d must be >= N=%d", name, p.ldc, p.N);
  NS2_REQUIRE(aligned16(p.A) && aligned16(p.W), "%s: A and W must be 16-byte aligned", name);
  NS2_REQUIRE(p.cOff >= 0 && p.gOff >= 0, "%s: negative offset", name);
  NS2_REQUIRE(p.act >= NS2_ACT_NONE && p.act <= NS2_ACT_GELU_TANH, "%s: unknown act %d", name, p.act);
  return NS2_OK;
}

template <int XFMT>
void launch_lora_down(const void* x, int ldx, const half_t* A, float* t, int M, int K, int R, hipStream_t s) {
  if (K % 32 == 0) {
    lora_down16_kernel<XFMT><<<dim3((M + 15) / 16, R / 32), 512, 0, s>>>(x, ldx, A, t, M, K, R);
    return;
  }
  const dim3 grid((M + 31) / 32);
  switch (R / 32) {
#define NS2_LORA_CASE(RT) \
  case RT: lora_down_kernel<XFMT, RT><<<grid, 64 * lora_waves<RT>(), 0, s>>>(x, ldx, A, t, M, K); break;
    NS2_LORA_CASE(1) NS2_LORA_CASE(2) NS2_LORA_CASE(3) NS2_LORA_CASE(4)
    NS2_LORA_CASE(5) NS2_LORA_CASE(6) NS2_LORA_CASE(7) NS2_LORA_CASE(8)
#undef NS2_LORA_CASE
    default: break;
  }
}

}  // namespace

namespace ns2 {

int lora_prepare(const float** t, const uint16_t* lora_a, const uint16_t* lora_b, int R, const void* x, int x_fmt,
                 int ldx, int M, int K, const char* name) {
  NS2_REQUIRE(lora_a && lora_b && aligned16(lora_a) && aligned16(lora_b), "%s: null or unaligned LoRA projections", name);
  NS2_REQUIRE(R > 0 && R % 32 == 0 && R <= 256,
              "%s: LoRA rank %d must be a positive multiple of 32, at most 256 (pad with zero rows)", name, R);
  NS2_REQUIRE(K % 16 == 0 && x && aligned16(x), "%s: LoRA input must be 16-byte aligned with K %% 16 == 0", name);
  NS2_REQUIRE(x_fmt == 2 || ldx % (x_fmt == 0 ? 4 : 8) == 0, "%s: LoRA input stride %d not 16-byte aligned", name, ldx);
  float* tb = static_cast<float*>(workspace(6, (size_t)M * R * sizeof(float)));
  if (!tb) return set_error(NS2_ERR_OOM, "%s: LoRA workspace allocation failed", name);
  ProfScope prof_("lora_down");
  const half_t* A = reinterpret_cast<const half_t*>(lora_a);
  if (x_fmt == 0) launch_lora_down<0>(x, ldx, A, tb, M, K, R, stream());
  else if (x_fmt == 1) launch_lora_down<1>(x, ldx, A, tb, M, K, R, stream());
  else launch_lora_down<2>(x, ldx, A, tb, M, K, R, stream());
  NS2_LAUNCHED("lora_down");
  *t = tb;
  return NS2_OK;
}

}  // namespace ns2

extern "C" {

int ns2_linear_i8(const void* A, int a_fmt, int lda, const int8_t* W, const float* scale,
                  const float* bias, const float* add, float* C, int M, int N, int K, int ldc,
                  long long cOff, float alpha, int act, int resid, const float* gate,
                  long long gOff) {
  return ns2_linear_i8_lora(A, a_fmt, lda, W, scale, bias, add, C, M, N, K, ldc, cOff, alpha, act, resid, gate,
                            gOff, nullptr, nullptr, 0);
}

int ns2_linear_i8_lora(const void* A, int a_fmt, int lda, const int8_t* W, const float* scale,
                       const float* bias, const float* add, float* C, int M, int N, int K, int ldc,
                       long long cOff, float alpha, int act, int resid, const float* gate,
                       long long gOff, const uint16_t* lora_a, const uint16_t* lora_b, int lora_r) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  GemmArgs p{A, W, scale, bias, add, C, gate, cOff, gOff, lda, ldc, M, N, K, alpha, act, resid};
  NS2_REQUIRE(a_fmt >= 0 && a_fmt <= 2,
              "ns2_linear_i8: a_fmt must be 0 (fp32), 1 (rotated fp16) or 2 (rotated fp32)");
  NS2_REQUIRE(scale != nullptr, "ns2_linear_i8: null scale");
  NS2_REQUIRE(K % 256 == 0, "ns2_linear_i8: K=%d must be a multiple of 256 (ConvRot groups)", K);
  if (a_fmt != 1) {
    // fp32 input: rotate (ops.linear without xr, app/gpu/ops.js:54) or just cast a
    // pre-rotated xr, into library scratch
    NS2_REQUIRE(A && lda >= K && lda % 4 == 0 && aligned16(A), "ns2_linear_i8: bad fp32 A / lda=%d", lda);
    uint16_t* xr = static_cast<uint16_t*>(ns2::workspace(0, (size_t)M * K * sizeof(uint16_t)));
    if (!xr) return ns2::set_error(NS2_ERR_OOM, "ns2_linear_i8: workspace allocation failed");
    if (a_fmt == 0) {
      int rc = ns2_rotate_f16(static_cast<const float*>(A), lda, xr, K, M, K, 0);
      if (rc) return rc;
    } else {
      const long long quads = (long long)M * K / 4;
      ns2::ProfScope prof_("cast_f16");
      cast_f16_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, ns2::stream()>>>(static_cast<const float*>(A), lda, xr, M, K);
      NS2_LAUNCHED("cast_f16");
    }
    p.A = xr;
    p.lda = K;
  }
  int rc = check_common(p, "ns2_linear_i8");
  if (rc) return rc;
  if (lora_r) {
    // the LoRA down-projections take the rotated input (rotated A for int8 weights)
    rc = ns2::lora_prepare(&p.lt, lora_a, lora_b, lora_r, p.A, 1, p.lda, M, K, "ns2_linear_i8_lora");
    if (rc) return rc;
    p.lb = reinterpret_cast<const half_t*>(lora_b);
    p.lr = lora_r;
  }
  return launch_gemm<false, false>(p, "linear_i8");
}

int ns2_linear_bf16(const float* A, int lda, const uint16_t* W, const float* bias,
                    const float* add, float* C, int M, int N, int K, int ldc, long long cOff,
                    float alpha, int act, int resid, const float* gate, long long gOff) {
  return ns2_linear_bf16_lora(A, lda, W, bias, add, C, M, N, K, ldc, cOff, alpha, act, resid, gate, gOff,
                              nullptr, nullptr, 0);
}

int ns2_linear_bf16_add_rmsnorm(const float* A, int lda, const uint16_t* W, const float* bias, float* x,
                                const float* w_add, const float* w_out, float* y, int M, int N, int K, float eps) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  NS2_REQUIRE(x && w_add && (!y || w_out), "ns2_linear_bf16_add_rmsnorm: null x, w_add or w_out");
  NS2_REQUIRE(N <= kRowNormMaxN, "ns2_linear_bf16_add_rmsnorm: N=%d exceeds %d", N, kRowNormMaxN);
  NS2_REQUIRE(y != x && A != x, "ns2_linear_bf16_add_rmsnorm: x must not alias A or y");
  // C is not written on this path (the row kernel writes x and y); x stands in for the check
  GemmArgs p{A, W, nullptr, bias, nullptr, x, nullptr, 0, 0, lda, N, M, N, K, 1.0f, NS2_ACT_NONE, 0};
  int rc = check_common(p, "ns2_linear_bf16_add_rmsnorm");
  if (rc) return rc;
  const RowNorm rn{x, w_add, w_out, y, eps};
  return launch_gemm<true, true>(p, "linear_bf16_add_rmsnorm", &rn);
}

int ns2_parts_add_rmsnorm(const float* part, int splits, const float* bias, float* x, const float* w_add,
                          const float* w_out, float* y, int M, int N, float eps) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  NS2_REQUIRE(part && x && w_add && (!y || w_out), "ns2_parts_add_rmsnorm: null part, x, w_add or w_out");
  NS2_REQUIRE(splits > 0 && M > 0 && N > 0 && N <= kRowNormMaxN, "ns2_parts_add_rmsnorm: splits=%d M=%d N=%d (N <= %d)",
              splits, M, N, kRowNormMaxN);
  NS2_REQUIRE(y != x && part != x, "ns2_parts_add_rmsnorm: x must not alias part or y");
  GemmArgs p{nullptr, nullptr, nullptr, bias, nullptr, x, nullptr, 0, 0, 0, N, M, N, 0, 1.0f, NS2_ACT_NONE, 0};
  p.part = const_cast<float*>(part);
  const RowNorm rn{x, w_add, w_out, y, eps};
  ns2::ProfScope prof_("parts_add_rmsnorm");
  launch_add_rmsnorm(p, splits, rn, ns2::stream());
  NS2_LAUNCHED("parts_add_rmsnorm");
  return NS2_OK;
}

namespace {

int linear_bf16_head_norm(const char* fn, const char* name, const float* A, int lda, const uint16_t* W, const float* bias, float* C,
                          int M, int N, int K, const float* w1, int H1, const float* w2, int H2, int D, const float* cs,
                          long long sin_off, int rope_rows, float eps, uint16_t* kv16, int ldkv) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  NS2_REQUIRE(D == 64 || D == 128 || D == 256, "%s: head dim %d is not 64, 128 or 256", fn, D);
  NS2_REQUIRE(N % D == 0 && N / D <= kHeadNormMaxHeads && H1 >= 0 && H2 >= 0 && (H1 + H2) * D <= N &&
                  (!H1 || w1) && (!H2 || w2),
              "%s: N=%d (at most %d heads of %d), H1=%d, H2=%d or their weights", fn, N, kHeadNormMaxHeads, D, H1,
              H2);
  NS2_REQUIRE(C != A, "%s: C must not alias A", fn);
  if (kv16) NS2_REQUIRE(ldkv >= N - H1 * D, "%s: ldkv=%d is below the %d fp16 key/value columns", fn, ldkv, N - H1 * D);
  GemmArgs p{A, W, nullptr, bias, nullptr, C, nullptr, 0, 0, lda, N, M, N, K, 1.0f, NS2_ACT_NONE, 0};
  int rc = check_common(p, fn);
  if (rc) return rc;
  const HeadNorm hn{w1, H1, w2, H2, D, cs, sin_off, cs ? rope_rows : 0, eps, reinterpret_cast<half_t*>(kv16), ldkv};
  return launch_gemm<true, true>(p, name, nullptr, nullptr, 0, &hn);
}

}  // namespace

int ns2_linear_bf16_head_norm(const float* A, int lda, const uint16_t* W, const float* bias, float* C, int M, int N,
                              int K, const float* w1, int H1, const float* w2, int H2, int D, const float* cs,
                              long long sin_off, int rope_rows, float eps) {
  return linear_bf16_head_norm("ns2_linear_bf16_head_norm", "linear_bf16_head_norm", A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D, cs,
                               sin_off, rope_rows, eps, nullptr, 0);
}

int ns2_linear_bf16_head_norm_f16kv(const float* A, int lda, const uint16_t* W, const float* bias, float* C, int M,
                                    int N, int K, const float* w1, int H1, const float* w2, int H2, int D,
                                    const float* cs, long long sin_off, int rope_rows, float eps, uint16_t* kv16,
                                    int ldkv) {
  NS2_READY();
  NS2_REQUIRE(kv16 || M == 0, "ns2_linear_bf16_head_norm_f16kv: null kv16");
  return linear_bf16_head_norm("ns2_linear_bf16_head_norm_f16kv", "linear_bf16_head_norm", A, lda, W, bias, C, M, N, K, w1, H1, w2, H2, D,
                               cs, sin_off, rope_rows, eps, kv16, ldkv);
}

int ns2_linear_bf16_glu(const float* A, int lda, const uint16_t* W, const float* bias, float* Y, int M, int N,
                        int K, int act) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  NS2_REQUIRE(Y && N % 2 == 0, "ns2_linear_bf16_glu: null Y or odd N=%d", N);
  NS2_REQUIRE(act >= NS2_ACT_NONE && act <= NS2_ACT_GELU_TANH, "ns2_linear_bf16_glu: unknown act %d", act);
  NS2_REQUIRE(Y != A, "ns2_linear_bf16_glu: Y must not alias A");
  // C is not written on this path (the GLU kernel writes Y); Y stands in for the check
  GemmArgs p{A, W, nullptr, bias, nullptr, Y, nullptr, 0, 0, lda, N, M, N, K, 1.0f, NS2_ACT_NONE, 0};
  int rc = check_common(p, "ns2_linear_bf16_glu");
  if (rc) return rc;
  return launch_gemm<true, true>(p, "linear_bf16_glu", nullptr, Y, act);
}

int ns2_linear_bf16_glu_down(const float* A, int lda, const uint16_t* W, const float* bias, int M, int N, int K,
                             int act, const uint16_t* wd_tiled, int Nd, float* part) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  const char* fn = "ns2_linear_bf16_glu_down";
  NS2_REQUIRE(wd_tiled && part, "%s: null wd_tiled or part", fn);
  NS2_REQUIRE(N % (2 * kGluDownGroup) == 0 && Nd > 0 && Nd % 64 == 0,
              "%s: N=%d must be a multiple of %d (%d-column GLU groups) and Nd=%d of 64", fn, N, 2 * kGluDownGroup,
              kGluDownGroup, Nd);
  NS2_REQUIRE(act >= NS2_ACT_NONE && act <= NS2_ACT_GELU_TANH, "%s: unknown act %d", fn, act);
  NS2_REQUIRE(aligned16(wd_tiled) && part != A, "%s: wd_tiled must be 16-byte aligned and part must not alias A", fn);
  // C is not written on this path; part stands in for the check
  GemmArgs p{A, W, nullptr, bias, nullptr, part, nullptr, 0, 0, lda, N, M, N, K, 1.0f, NS2_ACT_NONE, 0};
  int rc = check_common(p, fn);
  if (rc) return rc;
  const GluDown gd{reinterpret_cast<const half_t*>(wd_tiled), part, Nd, act, glu_down_ranges(M, N, Nd)};
  return launch_gemm<true, true>(p, "linear_bf16_glu_down", nullptr, nullptr, 0, nullptr, &gd);
}

int ns2_parts_add_rmsnorm_tiled(const float* part, int splits, const float* bias, float* x, const float* w_add,
                                const float* w_out, uint16_t* yt, int M, int N, float eps) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  const char* fn = "ns2_parts_add_rmsnorm_tiled";
  NS2_REQUIRE(part && x && w_add && w_out && yt, "%s: null part, x, w_add, w_out or yt", fn);
  NS2_REQUIRE(splits > 0 && M > 0 && N > 0 && N % 64 == 0 && N <= kRowNormMaxN,
              "%s: splits=%d M=%d N=%d (N %% 64 == 0, N <= %d)", fn, splits, M, N, kRowNormMaxN);
  NS2_REQUIRE(part != x && aligned16(yt), "%s: x must not alias part; yt 16-byte aligned", fn);
  GemmArgs p{nullptr, nullptr, nullptr, bias, nullptr, x, nullptr, 0, 0, 0, N, M, N, 0, 1.0f, NS2_ACT_NONE, 0};
  p.part = const_cast<float*>(part);
  const RowNorm rn{x, w_add, w_out, nullptr, eps, yt};
  ns2::ProfScope prof_("parts_add_rmsnorm");
  launch_add_rmsnorm(p, splits, rn, ns2::stream());
  NS2_LAUNCHED("parts_add_rmsnorm");
  return NS2_OK;
}

int ns2_linear_f16w_tiled_head_norm_f16kv(const uint16_t* At, const uint16_t* Wt, const float* bias, float* C, int M,
                                          int N, int K, const float* w1, int H1, const float* w2, int H2, int D,
                                          const float* cs, long long sin_off, int rope_rows, float eps,
                                          uint16_t* kv16, int ldkv) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  const char* fn = "ns2_linear_f16w_tiled_head_norm_f16kv";
  NS2_REQUIRE(C && kv16, "%s: null C or kv16", fn);
  NS2_REQUIRE(D == 64 || D == 128 || D == 256, "%s: head dim %d is not 64, 128 or 256", fn, D);
  NS2_REQUIRE(N % D == 0 && N / D <= kHeadNormMaxHeads && H1 >= 0 && H2 >= 0 && (H1 + H2) * D <= N &&
                  (!H1 || w1) && (!H2 || w2),
              "%s: N=%d (at most %d heads of %d), H1=%d, H2=%d or their weights", fn, N, kHeadNormMaxHeads, D, H1,
              H2);
  NS2_REQUIRE(ldkv >= N - H1 * D, "%s: ldkv=%d is below the %d fp16 key/value columns", fn, ldkv, N - H1 * D);
  float* part = nullptr;
  int splits = 1;
  int rc = ns2::linear_f16w_tiled_raw(fn, At, Wt, M, N, K, &part, &splits);
  if (rc) return rc;
  GemmArgs q{nullptr, nullptr, nullptr, bias, nullptr, C, nullptr, 0, 0, 0, N, M, N, K, 1.0f, NS2_ACT_NONE, 0};
  q.part = part;
  const HeadNorm hn{w1, H1, w2, H2, D, cs, sin_off, cs ? rope_rows : 0, eps, reinterpret_cast<half_t*>(kv16), ldkv};
  ns2::ProfScope prof_("head_norm_f16kv");
  hipStream_t s = ns2::stream();
  if (D == 64) splitk_head_norm_kernel<64><<<M, 64, 0, s>>>(q, splits, hn);
  else if (D == 128) splitk_head_norm_kernel<128><<<M, 128, 0, s>>>(q, splits, hn);
  else splitk_head_norm_kernel<256><<<M, 256, 0, s>>>(q, splits, hn);
  NS2_LAUNCHED("head_norm_f16kv");
  return NS2_OK;
}

int ns2_linear_f16w_tiled_glu_down(const uint16_t* At, const uint16_t* Wt, const float* bias, int M, int N, int K,
                                   int act, const uint16_t* wd_tiled, int Nd, float* part) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  const char* fn = "ns2_linear_f16w_tiled_glu_down";
  NS2_REQUIRE(wd_tiled && part, "%s: null wd_tiled or part", fn);
  NS2_REQUIRE(N % (2 * kGluDownGroup) == 0 && Nd > 0 && Nd % 64 == 0,
              "%s: N=%d must be a multiple of %d (%d-column GLU groups) and Nd=%d of 64", fn, N, 2 * kGluDownGroup,
              kGluDownGroup, Nd);
  NS2_REQUIRE(act >= NS2_ACT_NONE && act <= NS2_ACT_GELU_TANH, "%s: unknown act %d", fn, act);
  NS2_REQUIRE(aligned16(wd_tiled), "%s: wd_tiled must be 16-byte aligned", fn);
  float* gu = nullptr;
  int splits = 1;
  int rc = ns2::linear_f16w_tiled_raw(fn, At, Wt, M, N, K, &gu, &splits);
  if (rc) return rc;
  GemmArgs q{nullptr, nullptr, nullptr, bias, nullptr, part, nullptr, 0, 0, 0, N, M, N, K, 1.0f, NS2_ACT_NONE, 0};
  q.part = gu;
  const GluDown gd{reinterpret_cast<const half_t*>(wd_tiled), part, Nd, act, glu_down_ranges(M, N, Nd)};
  ns2::ProfScope prof_("glu_down");
  splitk_glu_down_kernel<kGluDownGroup>
      <<<dim3((M + 15) / 16, N / 2 / kGluDownGroup, gd.ncs), 512, 0, ns2::stream()>>>(q, splits, gd);
  NS2_LAUNCHED("glu_down");
  return NS2_OK;
}

int ns2_linear_bf16_lora(const float* A, int lda, const uint16_t* W, const float* bias,
                         const float* add, float* C, int M, int N, int K, int ldc, long long cOff,
                         float alpha, int act, int resid, const float* gate, long long gOff,
                         const uint16_t* lora_a, const uint16_t* lora_b, int lora_r) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  GemmArgs p{A, W, nullptr, bias, add, C, gate, cOff, gOff, lda, ldc, M, N, K, alpha, act, resid};
  int rc = check_common(p, "ns2_linear_bf16");
  if (rc) return rc;
  if (lora_r) {
    rc = ns2::lora_prepare(&p.lt, lora_a, lora_b, lora_r, A, 0, lda, M, K, "ns2_linear_bf16_lora");
    if (rc) return rc;
    p.lb = reinterpret_cast<const half_t*>(lora_b);
    p.lr = lora_r;
  }
  return launch_gemm<true, true>(p, "linear_bf16");
}

}  // extern "C"
