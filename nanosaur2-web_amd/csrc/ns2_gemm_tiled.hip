// int8 ConvRot linear on tiled operands: the DiT's fast path.
//
// Operand layouts (16-byte chunks; each 64x64 tile image is what one LDS stage holds per
// 64-row block):
//   A (rotated fp16 activations), written by the producing row kernel:
//     At[ceil(M/64)][K/64][8 k-chunks][64 rows][8 halfs]       (8 KB per 64x64 tile)
//   W (int8 ConvRot weights), re-tiled once after upload (ns2_tile_i8_weight), each byte
//   stored biased as u = w + 128:
//     Wt[N/64][K/64][8 k-chunks][64 rows][8 bytes]            (4 KB per 64x64 tile)
//   or W (bf16 weights of the plain linears), re-tiled once as fp16 (ns2_tile_bf16_weight) in
//   the layout of A:
//     Wt[N/64][K/64][8 k-chunks][64 rows][8 halfs]            (8 KB per 64x64 tile)
// Tiles move into LDS as 1 KB blocks with direct global->LDS copies (no registers, no LDS
// stores) into a ring of LDS stages, and the MFMA fragment reads are conflict-free: the 32
// lanes of a half-wave read 32 consecutive 16-byte (A) or 8-byte (W) rows. The int8
// weights are decoded to fp16 as they are read from LDS into the MFMA B operand (exact:
// half(0x6400 | u) - 1152 = w for |w| <= 128), and the per-output-row scale is applied in
// the epilogue, in the reference's order (app/gpu/gemm.js:159-164).
#include <type_traits>

#include "ns2_common.h"

using namespace ns2dev;

namespace {

struct TGemmArgs {
  const half_t* At;
  const uint8_t* Wt;
  const float* scale;
  const float* bias;
  float* C;
  uint16_t* Y;  // GLU epilogue: rotated fp16 output in the tiled layout, N/2 columns
  const float* gate;
  long long cOff, gOff;
  int M, N, K, ldc;
  int mblocks, nblocks;  // 64-row blocks of A (rounded up) and W
  int tiles_m, tiles_n;  // block tiles
  float alpha;
  int act, resid;
  // LoRA side path: lt fp32 [M][lr] (the down-projected input), lb fp16 [N][lr] (up-projections,
  // original row order, strengths folded), lr % 32 == 0; lr = 0 without LoRA
  const float* lt;
  const half_t* lb;
  int lr;
  // split-K (plain epilogue only): block (tile, z) sums k-tiles [z * ksplit, (z + 1) * ksplit)
  // into part[z] ([M, N] fp32, no epilogue); tiled_splitk_reduce_kernel adds the splits in z
  // order and applies the epilogue. part = nullptr: no split.
  float* part;
  int ksplit;
  // column bands of the tile order (block_tile): 1 keeps the row-group order
  int bands;
  // Packed attention values (plain store only): output columns [vcol0, vcol0 + heads * vD) are
  // written as fp16 into vpk in the flash kernel's value layout, [head][key tile][8 key chunks]
  // [vD][8] with vtiles 64-key tiles per head (key r = output row r), instead of into C.
  // vpk = nullptr: off. vcol0 and vD are multiples of 32 and M of 16.
  half_t* vpk;
  int vcol0, vD, vtiles;
};

// 8 biased bytes (two dwords) -> 8 halfs: byte u -> half(0x6400 | u) - 1152 = u - 128 = w.
// v_perm picks bytes of {x, 0x64646464}: selector bytes 4..7 are x's bytes, 0 is 0x64.
__device__ __forceinline__ half8_t u8x8_to_h8(uint2 w) {
  const half2_t off = {(half_t)1152.0f, (half_t)1152.0f};
  half8_t r;
  const uint32_t ws[2] = {w.x, w.y};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t lo = __builtin_amdgcn_perm(ws[i], 0x64646464u, 0x00050004u);
    const uint32_t hi = __builtin_amdgcn_perm(ws[i], 0x64646464u, 0x00070006u);
    const half2_t l = __builtin_bit_cast(half2_t, lo) - off;
    const half2_t h = __builtin_bit_cast(half2_t, hi) - off;
    r[4 * i + 0] = l[0];
    r[4 * i + 1] = l[1];
    r[4 * i + 2] = h[0];
    r[4 * i + 3] = h[1];
  }
  return r;
}

// One output: (acc * alpha) * rs + bi, activation, then store or add into the residual `old`
// (gated by gt) in the reference's order (app/gpu/gemm.js:159-164).
// Activation chosen at compile time (the launch dispatches on the argument).
template <int ACT>
__device__ __forceinline__ float act_t(float x) {
  if (ACT == NS2_ACT_SILU) return silu(x);
  if (ACT == NS2_ACT_GELU_TANH) return gelu_tanh(x);
  return x;
}

// XCD-aware tile order: consecutive block ids go to different XCDs (round-robin dispatch);
// block i is given tile start(x) + i/8 of XCD x = i % 8, where XCD x owns the contiguous range
// of T/8 (+1 for the first T%8 XCDs) tiles of a linear tile order, so neighbouring tiles
// (sharing A rows and W columns) run on the same XCD and meet in its L2. The linear order:
//  * bands > 1: column bands of ceil(tiles_n / bands) tiles, band by band, rows within a band,
//    N fastest. An XCD's range is then a 2-D block of one band, whose weight slice (sized on
//    the host to about half an L2) stays resident while its rows stream through once;
//  * bands = 1: N fastest inside groups of 4 row-tiles (A reuse in L2), for weights that fit.
__device__ __forceinline__ void block_tile(const TGemmArgs& p, int& tm, int& tn) {
  const int tiles = p.tiles_m * p.tiles_n;
  const int x = blockIdx.x % 8, local = blockIdx.x / 8;
  const int q = tiles / 8, rmd = tiles % 8;
  const int tile = x * q + (x < rmd ? x : rmd) + local;
  if (p.bands > 1) {
    const int bw = (p.tiles_n + p.bands - 1) / p.bands;
    const int band = tile / (bw * p.tiles_m), rem = tile % (bw * p.tiles_m);
    const int w = p.tiles_n - band * bw < bw ? p.tiles_n - band * bw : bw;  // the last band may be narrower
    tm = rem / w;
    tn = band * bw + rem % w;
    return;
  }
  const int group = 4;
  const int gsize = group * p.tiles_n;
  const int g = tile / gsize, rem = tile % gsize;
  const int rows_in_g = (p.tiles_m - g * group) < group ? (p.tiles_m - g * group) : group;
  tm = g * group + rem % rows_in_g;
  tn = rem / rows_in_g;
}

// Old outputs of a residual launch, loaded before the k loop (their latency hides behind it):
// cold[i][j][r] = C[mb + 32i + 8(r/4) + r%4][nb + 32j + lq].
template <int TM, int TN>
__device__ __forceinline__ void load_old(const TGemmArgs& p, float (&cold)[TM][TN][16], int mb, int nb, int lq) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = nb + 32 * j + lq;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mb + 32 * i + 8 * (r >> 2) + (r & 3);
        cold[i][j][r] = (m < p.M && n < p.N) ? p.C[p.cOff + (long long)m * p.ldc + n] : 0.0f;
      }
  }
}

// Plain epilogue of one wave (EPI 0): acc[i][j][r] = C[mb + 32i + 8(r/4) + r%4][nb + 32j + lq],
// mb = the wave's first row + 4hi. Per column: scale, bias, gate and the row-mb pointer; per
// element one multiply-add of its row offset and the arithmetic, with the row check only in
// tiles that cross M. RM 0 stores, RM 1 adds, RM 2 adds gate times the result
// (gemm.js:159-164); old outputs come from cold when PRE_C, else they are loaded here in a batch.
// LORA: the low-rank term of each tile (lora_tile) is added after the bias.
template <int TM, int TN, int ACT, int RM, bool PRE_C, bool LORA, int CI, int CJ>
__device__ __forceinline__ void store_plain(const TGemmArgs& p, const float16_t (&acc)[TM][TN],
                                            const float (&cold)[CI][CJ][16], int mb, int nb, bool full, int lq) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = nb + 32 * j + lq;
    if (n >= p.N) continue;
    const float rs = p.scale ? p.scale[n] : 1.0f;  // no per-row scale on fp16 weights
    const float bi = p.bias ? p.bias[n] : 0.0f;
    const float gt = RM == 2 ? p.gate[p.gOff + n] : 1.0f;
    float* cj = p.C + p.cOff + (long long)mb * p.ldc + n;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float16_t d;
      if constexpr (LORA) {
        const int hi = (mb & 4) ? 1 : 0;  // mb = the wave's first row + 4 hi (rows are 32-aligned)
        const int m = mb - 4 * hi + 32 * i + lq;
        d = lora_tile(p.lt, p.lb, p.lr, m < p.M ? m : p.M - 1, n, hi);
      }
      float old[16];
      if (RM != 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dm = 32 * i + 8 * (r >> 2) + (r & 3);
          old[r] = PRE_C ? cold[PRE_C ? i : 0][PRE_C ? j : 0][r]
                         : ((full || mb + dm < p.M) ? cj[(long long)dm * p.ldc] : 0.0f);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dm = 32 * i + 8 * (r >> 2) + (r & 3);
        if (!full && mb + dm >= p.M) continue;
        float v = acc[i][j][r] * p.alpha;
        v *= rs;
        v += bi;
        if constexpr (LORA) v += d[r];
        v = act_t<ACT>(v);
        if (RM == 1) v = old[r] + v;
        if (RM == 2) v = old[r] + gt * v;
        cj[(long long)dm * p.ldc] = v;
      }
    }
  }
}

// Plain store of one wave whose 32-column tiles lie in the packed-value window (RM 0): the
// values of the same epilogue, rounded to fp16 once, into the flash kernel's value layout. The
// 16 accumulator rows of a lane are keys {4hi..4hi+3, 8+4hi..8+4hi+3} of two 16-key groups,
// which the layout stores as one 16-byte chunk each (chunk 2g + hi of the group's 32 keys in
// a 64-key tile holds keys 16g + 4hi + {0..3} then 16g + 8 + 4hi + {0..3}).
template <int TM, int TN, int ACT, bool LORA>
__device__ __forceinline__ void store_vpack(const TGemmArgs& p, const float16_t (&acc)[TM][TN], int mb, int nb, int lq) {
  const int hi = (mb & 4) ? 1 : 0;  // mb = the wave's first row + 4 hi (rows are 32-aligned)
  const int m0 = mb - 4 * hi;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = nb + 32 * j + lq;
    const float rs = p.scale ? p.scale[n] : 1.0f;
    const float bi = p.bias ? p.bias[n] : 0.0f;
    const int c = n - p.vcol0, h = c / p.vD, dd = c % p.vD;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float16_t d;
      if constexpr (LORA) {
        const int m = m0 + 32 * i + lq;
        d = lora_tile(p.lt, p.lb, p.lr, m < p.M ? m : p.M - 1, n, hi);
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int key16 = m0 + 32 * i + 16 * g;
        if (key16 >= p.M) continue;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float x = acc[i][j][8 * g + e] * p.alpha;
          x *= rs;
          x += bi;
          if constexpr (LORA) x += d[8 * g + e];
          v[e] = act_t<ACT>(x);
          // the fp32 value first, as the plain store writes it: the conversion must not fuse
          // with the multiply-add into one rounding to fp16 (v_fma_mix)
          asm volatile("" : "+v"(v[e]));
        }
        const int kt = key16 >> 6, kc = 2 * ((key16 & 63) >> 4) + hi;
        half_t* dst = p.vpk + ((long long)h * p.vtiles + kt) * 64 * p.vD + ((long long)kc * p.vD + dd) * 8;
        uint4 q;
        q.x = pack_half2(v[0], v[1]);
        q.y = pack_half2(v[2], v[3]);
        q.z = pack_half2(v[4], v[5]);
        q.w = pack_half2(v[6], v[7]);
        *reinterpret_cast<uint4*>(dst) = q;
      }
    }
  }
}

// Block tile BM x BN (multiples of 64), BK = 64; WAVES_M x WAVES_N waves, each computing
// (BM/WAVES_M) x (BN/WAVES_N) with v_mfma_f32_32x32x16_f16 tiles. STAGES LDS stages, one
// barrier per k-tile: tile kt+STAGES-1 is copied in while tile kt is multiplied (with three
// stages the wait before the barrier leaves tile kt+1's copies in flight).
// EPI 0: C = act(A W^T * alpha * scale + bias) (RM 0), C += that (RM 1) or C += gate * that
// (RM 2), the order of gemm.js:159-164. EPI 1 (GLU): W's rows are interleaved in 32-row blocks
// (ns2_tile_i8_weight_glu), so the 64 columns of a wave hold 32 columns of each GLU half; the
// block's 512 columns give 256 consecutive outputs act(h1) * h2, one rotation group, which is
// rotated and written to Y as the tiled fp16 operand of the next int8 linear.
// WF16: fp16 weight tiles (the plain bf16 linears, re-tiled as fp16; no per-row scale unless
// given): 8 KB per 64x64 weight tile, read straight into the MFMA B operand.
// Waves per SIMD that a launch with the LoRA term keeps: the occupancy of the plain kernel of
// the same shape (left free, the compiler spends a few more registers on the LoRA variants and
// they lose a resident block: 128 -> 140 for the GLU launch).
template <int BM, int BN, int RM, bool LORA>
constexpr int lora_waves_per_eu() {
  if (!LORA) return 1;
  if (BM == 64 && BN == 512) return 4;
  if (BM == 64 && BN == 128) return RM ? 4 : 5;
  return 1;
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int EPI, int ACT, int RM, bool LORA, bool WF16 = false>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) __attribute__((amdgpu_waves_per_eu(lora_waves_per_eu<BM, BN, RM, LORA>())))
void gemm_tiled_kernel(TGemmArgs p) {
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int WCH = WF16 ? 8 : 4;  // 1 KB blocks per 64 weight rows of a k-tile
  constexpr int WB = WF16 ? 2 : 1;   // bytes per weight element
  constexpr int A_BLOCKS = BM / 64 * 8, W_BLOCKS = BN / 64 * WCH;  // 1 KB blocks per stage
  constexpr int BLOCKS = A_BLOCKS + W_BLOCKS;
  constexpr int PER_WAVE = BLOCKS / NW;
  static_assert(BM % 64 == 0 && BN % 64 == 0 && WTM % 32 == 0 && WTN % 32 == 0, "tile shape");
  static_assert(BLOCKS % NW == 0, "copies must split evenly over the waves");

  static_assert(STAGES == 2 || STAGES == 3, "two or three LDS stages");
  static_assert(!WF16 || EPI == 0, "fp16 weights take the plain epilogue");
  __shared__ __attribute__((aligned(16))) half_t as[STAGES][BM * 64];
  __shared__ __attribute__((aligned(16))) uint8_t ws[STAGES][BN * 64 * WB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int lq = lane & 31, hi = lane >> 5;

  int tm, tn;
  block_tile(p, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  // k-tiles of this block: all of K, or split z = blockIdx.y's range
  const int kt0 = p.part ? (int)blockIdx.y * p.ksplit : 0;
  const int kblocks = p.part ? (p.K / 64 - kt0 < p.ksplit ? p.K / 64 - kt0 : p.ksplit) : p.K / 64;
  const int kall = p.K / 64;
  // Stage image: A blocks (8 k-chunks of 1 KB per 64-row block), then W blocks (WCH per 64-row
  // block). Block ids past the last real 64-row block re-read the last one (their rows are
  // dropped). The per-wave sources and destinations are fixed up front; a k-tile adds its offset.
  const char* g_src[PER_WAVE];
  uint32_t l_dst[PER_WAVE];
  int g_step[PER_WAVE], l_step[PER_WAVE];
  {
    const uint32_t as_base = lds_addr(as), ws_base = lds_addr(ws);
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int j = wave + i * NW;
      if (j < A_BLOCKS) {
        const int mbi = j / 8, c = j % 8;
        int mb = m0 / 64 + mbi;
        mb = mb < p.mblocks ? mb : p.mblocks - 1;
        g_src[i] = reinterpret_cast<const char*>(p.At) + ((long long)mb * kall * 8 + (long long)kt0 * 8 + c) * 1024;
        l_dst[i] = as_base + j * 1024;
        g_step[i] = 8 * 1024;
        l_step[i] = BM * 64 * 2;
      } else {
        const int jw = j - A_BLOCKS;
        const int nbi = jw / WCH, c = jw % WCH;
        int nb = n0 / 64 + nbi;
        nb = nb < p.nblocks ? nb : p.nblocks - 1;
        g_src[i] = reinterpret_cast<const char*>(p.Wt) + ((long long)nb * kall * WCH + (long long)kt0 * WCH + c) * 1024;
        l_dst[i] = ws_base + jw * 1024;
        g_step[i] = WCH * 1024;
        l_step[i] = BN * 64 * WB;
      }
    }
  }
  auto dma = [&](int kt, int st) {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i)
      dma16(g_src[i] + (long long)kt * g_step[i] + lane * 16, __builtin_amdgcn_readfirstlane(l_dst[i] + st * l_step[i]));
  };

  float16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Residual launches of small wave tiles load their old outputs before the k loop, where the
  // latency hides behind it, instead of in the epilogue.
  constexpr bool PRE_C = EPI == 0 && RM != 0 && TM * TN * 16 <= 32;
  float cold[PRE_C ? TM : 1][PRE_C ? TN : 1][16];
  if constexpr (PRE_C) {
    if (!p.part) load_old<TM, TN>(p, cold, m0 + wm * WTM + 4 * hi, n0 + wn * WTN, lq);
  }

  dma(0, 0);
  if (STAGES == 3 && kblocks > 1) dma(1, 1);

  // fragments of k-step s (16 k) of a stage: A rows wm*WTM + 32i + lq, k 16s + 8hi .. +7 (chunk
  // 2s + hi); W columns wn*WTN + 32j + lq, the same k (8-byte chunk 2s + hi, or 16-byte chunk for
  // fp16 weights, read as the B operand itself)
  auto read_a = [&](int st, int s, int i) {
    const int row = wm * WTM + 32 * i;
    const int mbi = row / 64, r0 = row % 64;
    return *reinterpret_cast<const half8_t*>(&as[st][((mbi * 8 + 2 * s + hi) * 64 + r0 + lq) * 8]);
  };
  using WRaw = std::conditional_t<WF16, half8_t, uint2>;
  auto read_w = [&](int st, int s, int j) {
    const int col = wn * WTN + 32 * j;
    const int nbi = col / 64, c0 = col % 64;
    return *reinterpret_cast<const WRaw*>(&ws[st][((nbi * 8 + 2 * s + hi) * 64 + c0 + lq) * 8 * WB]);
  };
  auto decode = [&](const WRaw& w) {
    if constexpr (WF16) return w;
    else return u8x8_to_h8(w);
  };

  for (int kt = 0; kt < kblocks; ++kt) {
    const int st = kt % STAGES;
    // this wave's copies of tile kt have landed once at most tile kt+1's remain in flight
    // (three stages); the barrier then covers every wave's copies, and every wave's reads of
    // tile kt-1, whose stage the next copies overwrite
    if (STAGES == 3 && kt + 1 < kblocks) vm_wait<PER_WAVE>();
    else vm_wait<0>();
    __syncthreads();
    if (kt + STAGES - 1 < kblocks) dma(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
    __builtin_amdgcn_s_setprio(1);
    // k-steps of 16, software-pipelined: fragments read two steps ahead, the weights decoded
    // one step ahead, behind the MFMAs; scheduling barriers pin the order (the default
    // scheduler would put every read right before its use to save registers)
    half8_t a[3][TM], b[2][TN];
    WRaw w[3][TN];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int i = 0; i < TM; ++i) a[s][i] = read_a(st, s, i);
#pragma unroll
      for (int j = 0; j < TN; ++j) w[s][j] = read_w(st, s, j);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) b[0][j] = decode(w[0][j]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s + 2 < 4) {
#pragma unroll
        for (int i = 0; i < TM; ++i) a[(s + 2) % 3][i] = read_a(st, s + 2, i);
#pragma unroll
        for (int j = 0; j < TN; ++j) w[(s + 2) % 3][j] = read_w(st, s + 2, j);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[s % 3][i], b[s & 1][j], acc[i][j], 0, 0, 0);
      if (s + 1 < 4) {
#pragma unroll
        for (int j = 0; j < TN; ++j) b[(s + 1) & 1][j] = decode(w[(s + 1) % 3][j]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  }

  if constexpr (EPI == 1) {
    // ---- GLU + rotation epilogue (BM = 64, BN = 512, one wave row, 64 columns per wave)
    static_assert(BM == 64 && BN == 512 && WAVES_M == 1 && TM == 2 && TN == 2, "GLU epilogue tile");
    const int I = p.N / 2;
    const int gb = n0 / 2;            // first output (GLU) column of the block
    const int gc = 32 * wn + lq;      // this lane's output column within the block
    const int G = gb + gc;
    const float s1 = p.scale[G], s2 = p.scale[I + G];
    const float b1 = p.bias ? p.bias[G] : 0.0f, b2 = p.bias ? p.bias[I + G] : 0.0f;
    __syncthreads();  // every wave is done with the LDS stages
    float* T = reinterpret_cast<float*>(&ws[0][0]);  // [64 rows][256 columns] fp32 = the W stages
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (LORA) {
        // the low-rank terms of the two halves' tiles (weight rows G and I + G), one tile at a
        // time: act(h1) goes through T, then h2 multiplies it in place
        int m = m0 + 32 * i + lq;
        m = m < p.M ? m : p.M - 1;
        const float16_t d1 = lora_tile(p.lt, p.lb, p.lr, m, G, hi);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 32 * i + 8 * (r >> 2) + 4 * hi + (r & 3);
          float h1 = acc[i][0][r] * p.alpha;
          h1 *= s1;
          h1 += b1;
          T[row * 256 + gc] = act_t<ACT>(h1 + d1[r]);
        }
        const float16_t d2 = lora_tile(p.lt, p.lb, p.lr, m, I + G, hi);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 32 * i + 8 * (r >> 2) + 4 * hi + (r & 3);
          float h2 = acc[i][1][r] * p.alpha;
          h2 *= s2;
          h2 += b2;
          T[row * 256 + gc] *= h2 + d2[r];
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 32 * i + 8 * (r >> 2) + 4 * hi + (r & 3);
          // the linear's epilogue order (no activation there), then the GLU
          float h1 = acc[i][0][r] * p.alpha;
          h1 *= s1;
          h1 += b1;
          float h2 = acc[i][1][r] * p.alpha;
          h2 *= s2;
          h2 += b2;
          T[row * 256 + gc] = act_t<ACT>(h1) * h2;
        }
      }
    }
    __syncthreads();
    // rotation: wave w rotates rows 8w .. 8w+7 on the matrix cores, the fp16 result in place in
    // the first 512 bytes of the row, its 16-byte chunk c stored at chunk c ^ (row & 7): the
    // copy-out below reads one chunk of 64 rows 1 KB apart per wave, and the swizzle puts 8
    // consecutive rows in 8 different bank groups (unswizzled, all 64 lanes hit the same four
    // banks)
#pragma unroll
    for (int rr = 0; rr < 64 / NW; ++rr) {
      // the matrix-core FWHT: lane l holds columns lo .. lo+3, lo = 16(l%16) + 4(l/16)
      const half4v_t hf = fwht_h16_fragment();
      const int lo = fwht_mfma_offset();
      const int row = (64 / NW) * wave + rr;
      const float4 in = *reinterpret_cast<const float4*>(T + row * 256 + lo);
      float v[4] = {in.x, in.y, in.z, in.w};
      fwht256_mfma(v, hf);
      uint2 o;
      o.x = pack_half2(v[0], v[1]);
      o.y = pack_half2(v[2], v[3]);
      char* rb = reinterpret_cast<char*>(T + row * 256);
      *reinterpret_cast<uint2*>(rb + ((lo >> 3) ^ (row & 7)) * 16 + ((lo >> 2) & 1) * 8) = o;
    }
    __syncthreads();
    // 32 chunks of 8 columns x 64 rows: 1 KB contiguous each in the tiled layout
    for (int q = tid; q < 32 * 64; q += NW * 64) {
      const int row = q % 64, c = q / 64;
      const char* rb = reinterpret_cast<const char*>(T + row * 256);
      const uint4 v = *reinterpret_cast<const uint4*>(rb + (c ^ (row & 7)) * 16);
      *reinterpret_cast<uint4*>(p.Y + tiled_off(m0 + row, gb + c * 8, I)) = v;
    }
    return;
  }
  if (p.part) {
    // split-K: the raw partial products of split blockIdx.y
    float* part = p.part + (long long)blockIdx.y * p.M * p.N;
    const int mb = m0 + wm * WTM + 4 * hi, nb = n0 + wn * WTN;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = nb + 32 * j + lq;
      if (n >= p.N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = mb + 32 * i + 8 * (r >> 2) + (r & 3);
          if (m < p.M) part[(long long)m * p.N + n] = acc[i][j][r];
        }
    }
    return;
  }
  if (RM == 0 && p.vpk && n0 + wn * WTN >= p.vcol0 && n0 + wn * WTN < p.N) {
    store_vpack<TM, TN, ACT, LORA>(p, acc, m0 + wm * WTM + 4 * hi, n0 + wn * WTN, lq);
    return;
  }
  store_plain<TM, TN, ACT, RM, PRE_C, LORA>(p, acc, cold, m0 + wm * WTM + 4 * hi, n0 + wn * WTN, m0 + BM <= p.M, lq);
}

// The splits of a split-K launch summed in z order (deterministic), then the plain epilogue of
// store_plain (scale, bias, the LoRA term, activation, store / += / += gate times).
__global__ __launch_bounds__(256) void tiled_splitk_reduce_kernel(TGemmArgs p, int splits) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long mn = (long long)p.M * p.N;
  if (idx >= mn) return;
  float acc = 0.f;
  for (int z = 0; z < splits; ++z) acc += p.part[z * mn + idx];
  const int m = (int)(idx / p.N), n = (int)(idx % p.N);
  float v = acc * p.alpha;
  if (p.scale) v *= p.scale[n];
  v += p.bias ? p.bias[n] : 0.0f;
  if (p.lr) v += lora_dot(p.lt, p.lb, p.lr, m, n);
  if (p.act == NS2_ACT_SILU) v = silu(v);
  else if (p.act == NS2_ACT_GELU_TANH) v = gelu_tanh(v);
  float* c = p.C + p.cOff + (long long)m * p.ldc + n;
  if (!p.resid) *c = v;
  else if (!p.gate) *c = *c + v;
  else *c = *c + p.gate[p.gOff + n] * v;
}

// The same for launches with a LoRA term, one wave per 32x32 output tile: the lane sums the
// splits of its 16 elements (the v_mfma_f32_32x32x16_f16 accumulator layout, rows 8(r/4) +
// 4hi + r%4 of the tile, column lq), adds the tile's LoRA term on the matrix cores (lora_tile,
// as the unsplit epilogues do) and applies the epilogue. An element-wise reduce would take the
// LoRA term as R scalar products per element: 51.7 us for 256 x 3072 at rank 32.
__global__ __launch_bounds__(256) void tiled_splitk_reduce_lora_kernel(TGemmArgs p, int splits) {
  const int lane = threadIdx.x & 63, lq = lane & 31, hi = lane >> 5;
  const int tn_count = p.N / 32;
  const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tile >= ((p.M + 31) / 32) * tn_count) return;  // uniform per wave
  const int m0 = (tile / tn_count) * 32, n = (tile % tn_count) * 32 + lq;
  const long long mn = (long long)p.M * p.N;
  float acc[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + 8 * (r >> 2) + 4 * hi + (r & 3);
    float a = 0.f;
    if (m < p.M)
      for (int z = 0; z < splits; ++z) a += p.part[z * mn + (long long)m * p.N + n];
    acc[r] = a;
  }
  const int mrow = m0 + lq < p.M ? m0 + lq : p.M - 1;
  const float16_t d = lora_tile(p.lt, p.lb, p.lr, mrow, n, hi);
  const float rs = p.scale ? p.scale[n] : 1.0f;
  const float bi = p.bias ? p.bias[n] : 0.0f;
  const float gt = p.gate ? p.gate[p.gOff + n] : 1.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + 8 * (r >> 2) + 4 * hi + (r & 3);
    if (m >= p.M) continue;
    float v = acc[r] * p.alpha;
    v *= rs;
    v += bi;
    v += d[r];
    if (p.act == NS2_ACT_SILU) v = silu(v);
    else if (p.act == NS2_ACT_GELU_TANH) v = gelu_tanh(v);
    float* c = p.C + p.cOff + (long long)m * p.ldc + n;
    if (!p.resid) *c = v;
    else *c = *c + gt * v;
  }
}

// W [N, K] row-major int8 -> Wt tiles [N/64][K/64][8 k-chunks of 8][64 rows][8 bytes] of biased
// bytes (w + 128); one thread per 8-byte chunk.
__global__ __launch_bounds__(256) void tile_w_kernel(const int8_t* __restrict__ W, uint8_t* __restrict__ Wt,
                                                      int N, int K, int glu) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;  // output chunk index
  const long long chunks = (long long)N * K / 8;
  if (i >= chunks) return;
  // chunk order: [nb][kb][c 0..7][row 0..63]
  const int row = (int)(i % 64);
  const int c = (int)((i / 64) % 8);
  const long long rest = i / 512;  // nb * (K/64) + kb
  const int kb = (int)(rest % (K / 64));
  const int nb = (int)(rest / (K / 64));
  int n = nb * 64 + row;
  // GLU interleave: tiled row 64q + t holds row 32q + t of the first half (t < 32) or row
  // N/2 + 32q + t - 32 of the second half
  if (glu) n = row < 32 ? 32 * nb + row : N / 2 + 32 * nb + row - 32;
  uint2 v = *reinterpret_cast<const uint2*>(W + (long long)n * K + kb * 64 + c * 8);
  v.x ^= 0x80808080u;
  v.y ^= 0x80808080u;
  *reinterpret_cast<uint2*>(Wt + i * 8) = v;
}

// W [N, K] row-major bf16 -> Wt tiles [N/64][K/64][8 k-chunks of 8][64 rows][8 halfs] of fp16
// (round to nearest even, as the row-major kernel's loader converts them); one thread per
// 16-byte chunk.
__global__ __launch_bounds__(256) void tile_w16_kernel(const uint16_t* __restrict__ W, uint16_t* __restrict__ Wt,
                                                        int N, int K) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;  // output chunk index
  const long long chunks = (long long)N * K / 8;
  if (i >= chunks) return;
  const int row = (int)(i % 64);
  const int c = (int)((i / 64) % 8);
  const long long rest = i / 512;  // nb * (K/64) + kb
  const int kb = (int)(rest % (K / 64));
  const int nb = (int)(rest / (K / 64));
  const uint4 v = *reinterpret_cast<const uint4*>(W + (long long)(nb * 64 + row) * K + kb * 64 + c * 8);
  const uint32_t in[4] = {v.x, v.y, v.z, v.w};
  uint32_t out[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    out[j] = pack_half2(__builtin_bit_cast(float, in[j] << 16), __builtin_bit_cast(float, in[j] & 0xffff0000u));
  *reinterpret_cast<uint4*>(Wt + i * 8) = make_uint4(out[0], out[1], out[2], out[3]);
}

// Weight bytes per column band of the tile order: half of an XCD's 4 MB L2.
constexpr long long kBandBytes = 2ll << 20;

template <int BM, int BN, int WM, int WN, int STAGES = 2, int EPI = 0, bool WF16 = false>
int launch_tiled(TGemmArgs p, int splits = 1, bool reduce = true) {
  p.tiles_m = (p.M + BM - 1) / BM;
  p.tiles_n = (p.N + BN - 1) / BN;
  // column bands (1, 2, 4 or 8) by an estimate of the bytes the XCDs' L2s miss: with b bands
  // each of the 8 XCDs reads its rows of A (A b / 8 in all) and a 1/b slice of W, re-read about
  // twice when the slice exceeds kBandBytes and three times when it exceeds an L2 (the factors
  // fit FETCH_SIZE at the DiT shapes: 3952 rows x {4608, 1536, 8192} x {1536, 4096}). Launches
  // with a few row tiles read each weight tile about once whatever the order.
  p.bands = 1;
  if (p.tiles_m >= 8) {
    const double a_bytes = (double)p.tiles_m * BM * p.K * 2, w_bytes = (double)p.N * p.K * (WF16 ? 2 : 1);
    double best = 0;
    for (int b = 1; b <= 8 && b <= p.tiles_n; b *= 2) {
      const double slice = w_bytes / b;
      const double f = slice <= kBandBytes ? 1.0 : (slice <= 2 * kBandBytes ? 2.0 : 3.0);
      const double est = a_bytes * b + w_bytes * (8.0 / b) * f;
      if (b == 1 || est < best) {
        best = est;
        p.bands = b;
      }
    }
  }
  const dim3 grid(p.tiles_m * p.tiles_n, splits), block(WM * WN * 64);
  hipStream_t s = ns2::stream();
  const int rm = !p.resid ? 0 : (p.gate ? 2 : 1);
#define NS2_TILED(A, R)                                                                               \
  do {                                                                                                \
    if constexpr (BM * BN < 256 * 256) {                                                              \
      if (p.lr) {                                                                                     \
        gemm_tiled_kernel<BM, BN, WM, WN, STAGES, EPI, A, R, true, WF16><<<grid, block, 0, s>>>(p);   \
        break;                                                                                        \
      }                                                                                               \
    }                                                                                                 \
    gemm_tiled_kernel<BM, BN, WM, WN, STAGES, EPI, A, R, false, WF16><<<grid, block, 0, s>>>(p);      \
  } while (0)
  if constexpr (EPI == 1) {
    if (p.act == NS2_ACT_SILU) NS2_TILED(NS2_ACT_SILU, 0);
    else if (p.act == NS2_ACT_GELU_TANH) NS2_TILED(NS2_ACT_GELU_TANH, 0);
    else NS2_TILED(NS2_ACT_NONE, 0);
  } else {
    switch (p.act * 3 + rm) {
      case 0: NS2_TILED(NS2_ACT_NONE, 0); break;
      case 1: NS2_TILED(NS2_ACT_NONE, 1); break;
      case 2: NS2_TILED(NS2_ACT_NONE, 2); break;
      case 3: NS2_TILED(NS2_ACT_SILU, 0); break;
      case 4: NS2_TILED(NS2_ACT_SILU, 1); break;
      case 5: NS2_TILED(NS2_ACT_SILU, 2); break;
      case 6: NS2_TILED(NS2_ACT_GELU_TANH, 0); break;
      case 7: NS2_TILED(NS2_ACT_GELU_TANH, 1); break;
      default: NS2_TILED(NS2_ACT_GELU_TANH, 2); break;
    }
  }
#undef NS2_TILED
  NS2_LAUNCHED("gemm_tiled");
  if (p.part && reduce) {
    const long long mn = (long long)p.M * p.N;
    if (p.lr) {
      const long long tiles32 = (long long)((p.M + 31) / 32) * (p.N / 32);
      tiled_splitk_reduce_lora_kernel<<<(unsigned)((tiles32 + 3) / 4), 256, 0, s>>>(p, splits);
    } else {
      tiled_splitk_reduce_kernel<<<(unsigned)((mn + 255) / 256), 256, 0, s>>>(p, splits);
    }
    NS2_LAUNCHED("gemm_tiled_splitk_reduce");
  }
  return NS2_OK;
}

// Block-tile configurations: BM x BN, the waves' layout, and two
// throughput figures fitted to measurements at the DiT shapes (3952 x {4608, 1536, 8192} x
// {1536, 4096}, 256 x 3072 x 1536), in tile-area units per microsecond at K = 1536: `rate`
// with the CUs full, `alone` for a CU that runs a single tile of this shape.
struct TileCfg {
  int bm, bn;
  float rate, alone;
};
constexpr TileCfg kCfgs[] = {
    {256, 256, 1154.f, 1587.f},  // 16 waves (4 x 4) of 64x64, 96 KB LDS
    {64, 128, 950.f, 532.f},     // 4 waves (1 x 4) of 64x32, 32 KB: each weight fragment decoded once
    {64, 64, 350.f, 347.f},      // 4 waves (2 x 2) of 32x32, 36 KB (three stages): few rows (text tokens)
};
constexpr int kCUs = 256;

// Estimated time: the tiles the busiest CU runs times the tile area over the full-CU rate, but
// never less than one tile running alone. The configuration with the least estimate is used.
int pick_config(int M, int N) {
  int best = -1;
  double best_t = 0;
  for (int i = 0; i < (int)(sizeof(kCfgs) / sizeof(kCfgs[0])); ++i) {
    const TileCfg& c = kCfgs[i];
    const long long tiles = (long long)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
    const long long per_cu = (tiles + kCUs - 1) / kCUs;
    const double area = (double)c.bm * c.bn;
    double t = per_cu * area / c.rate;
    if (t < area / c.alone) t = area / c.alone;
    if (best < 0 || t < best_t) {
      best = i;
      best_t = t;
    }
  }
  return best;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

namespace {

// wf16: Wt holds fp16 weight tiles (ns2_tile_bf16_weight) and scale may be null; otherwise
// int8 ConvRot tiles with their per-row scales (K a whole number of rotation groups).
int linear_tiled(const char* fn, bool wf16, const uint16_t* At, const void* Wt, const float* scale, const float* bias,
                 float* C, int M, int N, int K, int ldc, long long cOff, float alpha, int act, int resid,
                 const float* gate, long long gOff, const uint16_t* lora_a, const uint16_t* lora_b, int lora_r,
                 uint16_t* vpk = nullptr, int vcol0 = 0, int vD = 0, int vtiles = 0) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  NS2_REQUIRE(At && Wt && (scale || wf16) && C, "%s: null At, Wt, scale or C", fn);
  const int kmul = wf16 ? 64 : 256;
  NS2_REQUIRE(M > 0 && N > 0 && N % 64 == 0 && K > 0 && K % kmul == 0,
              "%s: M=%d N=%d K=%d (N %% 64 == 0, K %% %d == 0 required)", fn, M, N, K, kmul);
  NS2_REQUIRE(ldc >= N && cOff >= 0 && gOff >= 0, "%s: bad ldc/offsets", fn);
  NS2_REQUIRE(aligned16(At) && aligned16(Wt), "%s: operands must be 16-byte aligned", fn);
  NS2_REQUIRE(act >= NS2_ACT_NONE && act <= NS2_ACT_GELU_TANH, "%s: unknown act %d", fn, act);
  TGemmArgs p{reinterpret_cast<const half_t*>(At), static_cast<const uint8_t*>(Wt), scale, bias, C, nullptr, gate,
              cOff, gOff, M, N, K, ldc, (M + 63) / 64, N / 64, 0, 0, alpha, act, resid};
  p.vpk = reinterpret_cast<half_t*>(vpk);
  p.vcol0 = vcol0;
  p.vD = vD;
  p.vtiles = vtiles;
  if (lora_r) {
    int rc = ns2::lora_prepare(&p.lt, lora_a, lora_b, lora_r, At, 2, K, M, K, fn);
    if (rc) return rc;
    p.lb = reinterpret_cast<const half_t*>(lora_b);
    p.lr = lora_r;
  }
  ns2::ProfScope prof_(wf16 ? "gemm_f16_tiled" : "gemm_i8_tiled");
  // the 256x256 tiles (16 waves, 128 registers each) have no room for the LoRA term's registers
  int cfg = pick_config(M, N);
  if (lora_r && cfg == 0) cfg = 1;
  // Few rows (the 256 text tokens): when the 64x128 tiles do not cover the CUs more than once,
  // 64x64 tiles, and when even those leave CUs idle, K split over blockIdx.y (reduced in a second
  // launch) into about 320 blocks, at least 8 k-tiles per split and at most 8 splits. The
  // weights of these launches come from HBM (each is read once per pass), so the splits hide
  // its latency; measured at 256 rows with weights cycled through 320 MB (us, before -> after):
  // 4608 x 1536 21.9 -> 17.8 (no split), 8192 x 1536 21.1 -> 18.8, 1536 x 1536 with += 13.0 ->
  // 12.3 (3 splits), 1536 x 4096 with += 17.2 -> 16.8 (6 splits; 8 now).
  int splits = 1;
  if (cfg == 1 && (long long)((M + 63) / 64) * ((N + 127) / 128) <= kCUs) cfg = 2;
  if (cfg != 0) {
    const int bm = 64, bn = cfg == 1 ? 128 : 64;
    const long long tiles = (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int kt = K / 64;
    if (tiles < kCUs && kt >= 16 && !vpk) {
      splits = (int)((320 + tiles / 2) / tiles);
      if (splits > kt / 8) splits = kt / 8;
      if (splits > 8) splits = 8;
      if (splits < 1) splits = 1;
    }
    if (splits > 1) {
      p.ksplit = (kt + splits - 1) / splits;
      splits = (kt + p.ksplit - 1) / p.ksplit;
      p.part = static_cast<float*>(ns2::workspace(5, (size_t)splits * M * N * sizeof(float)));
      if (!p.part) return ns2::set_error(NS2_ERR_OOM, "%s: split-K workspace allocation failed", fn);
    }
  }
  if (wf16) {
    switch (cfg) {
      case 0: return launch_tiled<256, 256, 4, 4, 2, 0, true>(p);
      case 1: return launch_tiled<64, 128, 1, 4, 2, 0, true>(p, splits);
      default: return launch_tiled<64, 64, 2, 2, 2, 0, true>(p, splits);
    }
  }
  switch (cfg) {
    case 0: return launch_tiled<256, 256, 4, 4>(p);
    case 1:
      // at most two blocks per CU (2432 x 1536 launches: 456 tiles) the copies' latency shows, and
      // a third stage (48 KB, three blocks still fit) hides it: 2432 x 1536 x 6144 72.3 -> 69.6 us;
      // at three blocks per CU (the DiT's 744-tile proj and w3) it costs more than it hides
      if ((long long)((M + 63) / 64) * ((N + 127) / 128) <= 2 * kCUs) return launch_tiled<64, 128, 1, 4, 3>(p, splits);
      return launch_tiled<64, 128, 1, 4>(p, splits);
    // three stages: at a few rows each block runs alone on its CU and its weights come from HBM,
    // so a deeper copy queue pays (text q/k/v 22.0 -> 17.0 us, text proj 15.4 -> 14.3 us in the
    // pass); LDS is no limit at one block per CU
    default: return launch_tiled<64, 64, 2, 2, 3>(p, splits);
  }
}

}  // namespace

int ns2::linear_f16w_tiled_raw(const char* fn, const uint16_t* At, const uint16_t* Wt, int M, int N, int K,
                               float** part, int* splits) {
  NS2_REQUIRE(At && Wt && M > 0 && N > 0 && N % 64 == 0 && K > 0 && K % 64 == 0 && aligned16(At) && aligned16(Wt),
              "%s: At, Wt, M=%d, N=%d (N %% 64 == 0), K=%d (K %% 64 == 0) or alignment", fn, M, N, K);
  TGemmArgs p{reinterpret_cast<const half_t*>(At), reinterpret_cast<const uint8_t*>(Wt), nullptr, nullptr, nullptr,
              nullptr, nullptr, 0, 0, M, N, K, N, (M + 63) / 64, N / 64, 0, 0, 1.0f, NS2_ACT_NONE, 0};
  // 64x64 tiles (the few-row launches this serves); K split until about one block per CU, at
  // least 4 k-tiles per split
  const long long tiles = (long long)((M + 63) / 64) * (N / 64);
  const int kt = K / 64;
  int s = (int)(kCUs / tiles);
  if (s > kt / 4) s = kt / 4;
  if (s > 8) s = 8;
  if (s < 1) s = 1;
  p.ksplit = (kt + s - 1) / s;
  s = (kt + p.ksplit - 1) / p.ksplit;
  p.part = static_cast<float*>(ns2::workspace(5, (size_t)s * M * N * sizeof(float)));
  if (!p.part) return ns2::set_error(NS2_ERR_OOM, "%s: split-K workspace allocation failed", fn);
  *part = p.part;
  *splits = s;
  ns2::ProfScope prof_("gemm_f16_tiled");
  return launch_tiled<64, 64, 2, 2, 3, 0, true>(p, s, false);
}

extern "C" {

int ns2_tile_i8_weight(const int8_t* W, int8_t* Wt, int N, int K) {
  NS2_READY();
  NS2_REQUIRE(W && Wt && aligned16(W) && aligned16(Wt), "ns2_tile_i8_weight: null or unaligned buffer");
  NS2_REQUIRE(N > 0 && K > 0 && N % 64 == 0 && K % 64 == 0,
              "ns2_tile_i8_weight: N=%d and K=%d must be multiples of 64", N, K);
  const long long chunks = (long long)N * K / 8;
  ns2::ProfScope prof_("tile_i8_weight");
  tile_w_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, ns2::stream()>>>(W, reinterpret_cast<uint8_t*>(Wt), N, K, 0);
  NS2_LAUNCHED("tile_i8_weight");
  return NS2_OK;
}

int ns2_tile_i8_weight_glu(const int8_t* W, int8_t* Wt, int N, int K) {
  NS2_READY();
  NS2_REQUIRE(W && Wt && aligned16(W) && aligned16(Wt), "ns2_tile_i8_weight_glu: null or unaligned buffer");
  NS2_REQUIRE(N > 0 && K > 0 && N % 64 == 0 && K % 64 == 0,
              "ns2_tile_i8_weight_glu: N=%d and K=%d must be multiples of 64", N, K);
  const long long chunks = (long long)N * K / 8;
  ns2::ProfScope prof_("tile_i8_weight");
  tile_w_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, ns2::stream()>>>(W, reinterpret_cast<uint8_t*>(Wt), N, K, 1);
  NS2_LAUNCHED("tile_i8_weight_glu");
  return NS2_OK;
}

int ns2_linear_i8_glu_rot_tiled(const uint16_t* At, const int8_t* Wt, const float* scale, const float* bias,
                                uint16_t* Y, int M, int N, int K, float alpha, int act) {
  return ns2_linear_i8_glu_rot_tiled_lora(At, Wt, scale, bias, Y, M, N, K, alpha, act, nullptr, nullptr, 0);
}

int ns2_linear_i8_glu_rot_tiled_lora(const uint16_t* At, const int8_t* Wt, const float* scale, const float* bias,
                                     uint16_t* Y, int M, int N, int K, float alpha, int act, const uint16_t* lora_a,
                                     const uint16_t* lora_b, int lora_r) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  NS2_REQUIRE(At && Wt && scale && Y, "ns2_linear_i8_glu_rot_tiled: null At, Wt, scale or Y");
  NS2_REQUIRE(M > 0 && N > 0 && N % 512 == 0 && K > 0 && K % 256 == 0,
              "ns2_linear_i8_glu_rot_tiled: M=%d N=%d K=%d (N %% 512 == 0, K %% 256 == 0 required)", M, N, K);
  NS2_REQUIRE(aligned16(At) && aligned16(Wt) && aligned16(Y), "ns2_linear_i8_glu_rot_tiled: operands must be 16-byte aligned");
  NS2_REQUIRE(act >= NS2_ACT_NONE && act <= NS2_ACT_GELU_TANH, "ns2_linear_i8_glu_rot_tiled: unknown act %d", act);
  TGemmArgs p{reinterpret_cast<const half_t*>(At), reinterpret_cast<const uint8_t*>(Wt), scale, bias, nullptr, Y,
              nullptr, 0, 0, M, N, K, N, (M + 63) / 64, N / 64, 0, 0, alpha, act, 0};
  if (lora_r) {
    int rc = ns2::lora_prepare(&p.lt, lora_a, lora_b, lora_r, At, 2, K, M, K, "ns2_linear_i8_glu_rot_tiled_lora");
    if (rc) return rc;
    p.lb = reinterpret_cast<const half_t*>(lora_b);
    p.lr = lora_r;
  }
  ns2::ProfScope prof_("gemm_i8_glu_rot");
  return launch_tiled<64, 512, 1, 8, 2, 1>(p);
}

int ns2_linear_i8_tiled(const uint16_t* At, const int8_t* Wt, const float* scale, const float* bias,
                        float* C, int M, int N, int K, int ldc, long long cOff, float alpha, int act,
                        int resid, const float* gate, long long gOff) {
  return linear_tiled("ns2_linear_i8_tiled", false, At, Wt, scale, bias, C, M, N, K, ldc, cOff, alpha, act, resid, gate,
                         gOff, nullptr, nullptr, 0);
}

int ns2_linear_i8_tiled_lora(const uint16_t* At, const int8_t* Wt, const float* scale, const float* bias,
                             float* C, int M, int N, int K, int ldc, long long cOff, float alpha, int act,
                             int resid, const float* gate, long long gOff, const uint16_t* lora_a,
                             const uint16_t* lora_b, int lora_r) {
  return linear_tiled("ns2_linear_i8_tiled_lora", false, At, Wt, scale, bias, C, M, N, K, ldc, cOff, alpha, act, resid,
                         gate, gOff, lora_a, lora_b, lora_r);
}

int ns2_tile_bf16_weight(const uint16_t* W, uint16_t* Wt, int N, int K) {
  NS2_READY();
  NS2_REQUIRE(W && Wt && aligned16(W) && aligned16(Wt), "ns2_tile_bf16_weight: null or unaligned buffer");
  NS2_REQUIRE(N > 0 && K > 0 && N % 64 == 0 && K % 64 == 0,
              "ns2_tile_bf16_weight: N=%d and K=%d must be multiples of 64", N, K);
  const long long chunks = (long long)N * K / 8;
  ns2::ProfScope prof_("tile_bf16_weight");
  tile_w16_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, ns2::stream()>>>(W, Wt, N, K);
  NS2_LAUNCHED("tile_bf16_weight");
  return NS2_OK;
}

int ns2_linear_f16w_tiled(const uint16_t* At, const uint16_t* Wt, const float* bias, float* C, int M, int N, int K,
                          int ldc, long long cOff, float alpha, int act, int resid, const float* gate, long long gOff) {
  return linear_tiled("ns2_linear_f16w_tiled", true, At, Wt, nullptr, bias, C, M, N, K, ldc, cOff, alpha, act, resid,
                      gate, gOff, nullptr, nullptr, 0);
}

int ns2_linear_f16w_tiled_lora(const uint16_t* At, const uint16_t* Wt, const float* bias, float* C, int M, int N,
                               int K, int ldc, long long cOff, float alpha, int act, int resid, const float* gate,
                               long long gOff, const uint16_t* lora_a, const uint16_t* lora_b, int lora_r) {
  return linear_tiled("ns2_linear_f16w_tiled_lora", true, At, Wt, nullptr, bias, C, M, N, K, ldc, cOff, alpha, act,
                      resid, gate, gOff, lora_a, lora_b, lora_r);
}

int ns2_linear_i8_tiled_vpack(const uint16_t* At, const int8_t* Wt, const float* scale, const float* bias,
                              float* C, int M, int N, int K, int ldc, long long cOff, float alpha, int act,
                              const uint16_t* lora_a, const uint16_t* lora_b, int lora_r, uint16_t* vpk,
                              int vcol0, int H, int D, int Lk) {
  NS2_READY();
  if (M == 0) return NS2_OK;
  NS2_REQUIRE(vpk && ((uintptr_t)vpk & 15) == 0, "ns2_linear_i8_tiled_vpack: null or unaligned vpk");
  NS2_REQUIRE(H > 0 && D > 0 && D % 32 == 0 && vcol0 >= 0 && vcol0 % 64 == 0 && vcol0 + (long long)H * D == N,
              "ns2_linear_i8_tiled_vpack: the value columns [vcol0, vcol0 + H*D) must end the output "
              "(vcol0=%d H=%d D=%d N=%d; vcol0 %% 64 == 0, D %% 32 == 0)", vcol0, H, D, N);
  NS2_REQUIRE(M % 16 == 0 && M <= Lk, "ns2_linear_i8_tiled_vpack: M=%d must be a multiple of 16 and at most Lk=%d",
              M, Lk);
  return linear_tiled("ns2_linear_i8_tiled_vpack", false, At, Wt, scale, bias, C, M, N, K, ldc, cOff, alpha, act, 0,
                         nullptr, 0, lora_a, lora_b, lora_r, vpk, vcol0, D, (Lk + 63) / 64);
}

}  // extern "C"
