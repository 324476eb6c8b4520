// Internal helpers shared by the ns2 HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ns2.h"

namespace ns2 {

// ---- host side -------------------------------------------------------------------------

// Record an error message for ns2_last_error() and return code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
hipStream_t stream();
bool initialised();
// Stream-ordered scratch owned by the library, grown on demand and reused by later calls
// (one slot per concurrent use inside a single entry point).
void* workspace(int slot, size_t bytes);
constexpr int kWorkspaceSlots = 7;
// Device address of the current device's copy of the fixed scratch array that the
// allocation-free entry points use (NS2_NOALLOC_SCRATCH_BYTES bytes, resolved by ns2_init), or
// null before ns2_init has run on that device.
void* noalloc_scratch();
// LoRA side path of a linear: checks the stacked down/up projections (lora_a fp16 [R][K],
// lora_b fp16 [N][R], R % 32 == 0, R <= 256) and computes *t = x lora_a^T (fp32 [M][R], library
// scratch) from the linear's input x: x_fmt 0 fp32 [M][ldx], 1 fp16 [M][ldx], 2 fp16 in the
// tiled operand layout of the int8 GEMM (K columns). Returns a status code.
int lora_prepare(const float** t, const uint16_t* lora_a, const uint16_t* lora_b, int R, const void* x, int x_fmt,
                 int ldx, int M, int K, const char* name);
// The tiled linear over a re-tiled fp16 weight without its epilogue: the raw products of At Wt^T
// split over K into *splits fp32 partials *part ([*splits][M][N], library scratch slot 5, summed
// in split order by the caller's row kernel). At fp16 tiled [ceil(M/64)*64][K]. Returns a status code.
int linear_f16w_tiled_raw(const char* fn, const uint16_t* At, const uint16_t* Wt, int M, int N, int K, float** part,
                          int* splits);

// Kernel profiler (ns2_profile_*): when enabled, stream events bracket every launch and are
// aggregated by kernel name on ns2_profile_report.
void prof_begin(const char* name);
void prof_end();
struct ProfScope {
  explicit ProfScope(const char* name) { prof_begin(name); }
  ~ProfScope() { prof_end(); }
};

}  // namespace ns2

#define NS2_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ns2::set_error(NS2_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define NS2_HIP(expr)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                               \
      return ns2::set_error(NS2_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));      \
  } while (0)

#define NS2_LAUNCHED(name)                                                              \
  do {                                                                                  \
    hipError_t e_ = hipGetLastError();                                                  \
    if (e_ != hipSuccess)                                                               \
      return ns2::set_error(NS2_ERR_HIP, "launch %s: %s", name, hipGetErrorString(e_)); \
  } while (0)

#define NS2_READY()                                                             \
  do {                                                                          \
    if (!ns2::initialised())                                                    \
      return ns2::set_error(NS2_ERR_STATE, "ns2_init has not been called");      \
  } while (0)

// ---- device side -------------------------------------------------------------------------

typedef _Float16 half_t;
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef float float4_t __attribute__((ext_vector_type(4)));

namespace ns2dev {

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

// tanh-approximated GELU (PyTorch approximate="tanh"), tanh from exp of -2|u| so it
// cannot overflow (kernels.js:11-17).
__device__ __forceinline__ float gelu_tanh(float x) {
  float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  float e = __expf(-2.0f * fabsf(u));
  float t = copysignf((1.0f - e) / (1.0f + e), u);
  return 0.5f * x * (1.0f + t);
}

__device__ __forceinline__ float apply_act(float x, int act) {
  if (act == NS2_ACT_SILU) return silu(x);
  if (act == NS2_ACT_GELU_TANH) return gelu_tanh(x);
  return x;
}


// ---- in-wave fast Walsh-Hadamard transform (no LDS traffic) ----------------------------------
//
// The regular Hadamard H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] (tools/quant.py:25)
// maps x to y_i = (x_i + x_{i^1}) + (x_{i^2} - x_{i^3}): with T_i = x_i + x_{i^1} and
// E_j = x_j - x_{j^1}, y_i = T_i + E_{i^2}. Each radix-4 stage below evaluates that over the
// 4 values that differ in two index bits, held in registers or in lanes.

// DPP controls: quad_perm [1,0,3,2] (lane ^ 1), [2,3,0,1] (lane ^ 2), [3,2,1,0] (lane ^ 3);
// row_mirror (lane ^ 15 inside a row of 16); row_half_mirror (lane ^ 7 inside 8 lanes).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppXor3 = 0x1B, kDppRowMirror = 0x140,
              kDppHalfMirror = 0x141;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Stage over lane bits 0-1 (element stride 4): quad permutations.
__device__ __forceinline__ float h4_bits01(float v) {
  const float o = dpp<kDppXor1>(v);
  const float t = v + o, e = v - o;
  return t + dpp<kDppXor2>(e);
}

// Stage over lane bits 2-3 (stride 16): lane ^ 4 = half-row mirror then quad ^ 3, lane ^ 8 =
// row mirror then half-row mirror.
__device__ __forceinline__ float h4_bits23(float v) {
  const float o = dpp<kDppXor3>(dpp<kDppHalfMirror>(v));
  const float t = v + o, e = v - o;
  return t + dpp<kDppHalfMirror>(dpp<kDppRowMirror>(e));
}

// v_permlane16_swap / v_permlane32_swap (gfx950) as inline assembly: both registers are
// outputs, and the compiler's builtin returns the first operand's new value for both. The
// s_nop gives the two wait states these instructions need after a VALU write of an operand.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
#pragma clang diagnostic pop

// Sum over the 64 lanes of a wave, every lane gets it, without LDS traffic: quad sums by DPP
// (lane ^ 1, ^ 2), then the other quad of the 8-lane half row (half-row mirror), the other
// half of the 16-lane row (row mirror), the other row of the pair and the other 32-lane half
// (row swaps).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  {
    float a = v, b = v;
    permlane16_swap(a, b);  // {r0, r0, r2, r2}, {r1, r1, r3, r3}
    v = a + b;
  }
  {
    float a = v, b = v;
    permlane32_swap(a, b);  // {h0, h0}, {h1, h1}
    v = a + b;
  }
  return v;
}

// Block-wide sum for blockDim.x == 64 * nwaves (<= 1024); every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();  // red may still be read by a previous call
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// Stage over lane bits 4-5 (stride 64), with the row swaps. permlane16_swap exchanges the odd
// 16-lane rows of its first operand with the even rows of its second: on two copies of v (rows
// r0..r3) it leaves {r0, r0, r2, r2} and {r1, r1, r3, r3}, so every row holds its pair sum T
// and the difference (even - odd) of its pair. permlane32_swap does the same with 32-lane
// halves and leaves {lower half twice} and {upper half twice}: row i then takes the other
// half's difference, with the sign of x_{i^2} - x_{i^3} (negative on odd rows).
__device__ __forceinline__ float h4_bits45(float v) {
  float ev = v, od = v;
  permlane16_swap(ev, od);
  const float t = ev + od;
  float lo = ev - od, hi = lo;
  permlane32_swap(lo, hi);
  const float other = (threadIdx.x & 32) ? lo : hi;
  return __builtin_fmaf((threadIdx.x & 16) ? -1.0f : 1.0f, other, t);
}

// y = x H over one 256-group with H = kron(H4, H4, H4, H4) / 16 (tools/quant.py:21-29): lane t
// holds elements 4t..4t+3 in v[0..3]; stride 1 in registers, strides 4, 16 and 64 across
// lane bits 0-1, 2-3 and 4-5.
__device__ __forceinline__ void fwht256_wave(float v[4]) {
  {
    const float t01 = v[0] + v[1], e01 = v[0] - v[1], t23 = v[2] + v[3], e23 = v[2] - v[3];
    v[0] = t01 + e23;
    v[1] = t01 - e23;
    v[2] = t23 + e01;
    v[3] = t23 - e01;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = h4_bits01(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = h4_bits23(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = h4_bits45(v[j]) * 0.0625f;
}

// ---- FWHT of a 256-group on the matrix cores -----------------------------------------------
//
// With i = 16a + b, H256 = kron(H16, H16) / 16 for H16 = kron(H4, H4) (tools/quant.py:21-29), so
// y = x H256 is Y = H X H with X[a][b] = x[16a + b], Y[c][d] = y[16c + d] and H = H16 / 4.
// Two v_mfma_f32_16x16x16_f16 per factor: Z = X H, then Y^T = Z^T H. The lane layout of a
// 16x16x16 product (A[l%16][4(l/16)+j], B[4(l/16)+j][l%16], D[4(l/16)+j][l%16]) makes Z's
// accumulators exactly the A operand Z^T of the second product, and leaves Y^T's
// accumulators in the input layout: lane l holds elements 16(l%16) + 4(l/16) + j, j < 4.
// Each fp32 operand goes in as an fp16 pair hi + lo (two products accumulated in fp32; H's
// entries are +-1/4, exact), so the result keeps fp32 accuracy (~2^-21 relative).
typedef _Float16 half4v_t __attribute__((ext_vector_type(4)));

// H's B-operand fragment of this lane: H[4(l/16)+j][l%16] (H is symmetric, so it also serves
// as the A fragment H[l%16][4(l/16)+j] up to the transposition the layout already applies).
__device__ __forceinline__ half4v_t fwht_h16_fragment() {
  const int l = threadIdx.x & 63, n = l & 15;
  half4v_t h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k = 4 * (l >> 4) + j;
    // H4[p][q] = -1 where p + q = 3, else 1; H16[k][n] = H4[k/4][n/4] * H4[k%4][n%4]
    const int neg = ((k >> 2) + (n >> 2) == 3) ^ ((k & 3) + (n & 3) == 3);
    h[j] = (half_t)(neg ? -0.25f : 0.25f);
  }
  return h;
}

__device__ __forceinline__ void split_f16(const float v[4], half4v_t& hi, half4v_t& lo) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hi[j] = (half_t)v[j];
    lo[j] = (half_t)(v[j] - (float)hi[j]);
  }
}

// In place on v[4] in the layout above (lane l: elements 16(l%16) + 4(l/16) + j).
__device__ __forceinline__ void fwht256_mfma(float v[4], const half4v_t& h) {
  half4v_t hi, lo;
  split_f16(v, hi, lo);
  float4_t z = {0.f, 0.f, 0.f, 0.f};
  z = __builtin_amdgcn_mfma_f32_16x16x16f16(hi, h, z, 0, 0, 0);
  z = __builtin_amdgcn_mfma_f32_16x16x16f16(lo, h, z, 0, 0, 0);
  const float zv[4] = {z[0], z[1], z[2], z[3]};
  split_f16(zv, hi, lo);
  float4_t y = {0.f, 0.f, 0.f, 0.f};
  y = __builtin_amdgcn_mfma_f32_16x16x16f16(hi, h, y, 0, 0, 0);
  y = __builtin_amdgcn_mfma_f32_16x16x16f16(lo, h, y, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = y[j];
}

// First element of this lane's 4 in the matrix-core FWHT layout.
__device__ __forceinline__ int fwht_mfma_offset() {
  const int l = threadIdx.x & 63;
  return 16 * (l & 15) + 4 * (l >> 4);
}

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  half2_t h;
  h[0] = (half_t)a;
  h[1] = (half_t)b;
  return __builtin_bit_cast(uint32_t, h);
}

// Offset (in halfs) of element (m, k) of an fp16 GEMM operand with K columns in the tiled
// layout of the int8 GEMM: [M/64][K/64][8 k-chunks][64 rows][8 halfs] (ns2_linear_i8_tiled).
__device__ __forceinline__ long long tiled_off(long long m, int k, int K) {
  return (((m >> 6) * (K >> 6) + (k >> 6)) * 8 + ((k & 63) >> 3)) * 512 + (m & 63) * 8 + (k & 7);
}

// LDS byte address of a pointer into a __shared__ array, as a wave-uniform value.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p)));
}

// Direct global->LDS copy of 16 bytes per lane: lane l's bytes land at LDS address
// lds + 16 * l. Issued as inline assembly so that the compiler tracks neither the LDS
// write nor the load counter (it would otherwise wait for every outstanding copy before
// any LDS read): the caller waits with vm_wait<n>() and a barrier before reading the data.
// M0 carries the LDS base; no other code in the kernels that use this sets M0. An LDS DMA
// that reads M0 needs one wait state after the SALU write of M0 (the compiler's hazard
// rule for this generation, which it cannot apply inside an asm statement): s_nop 0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N vector-memory loads of this wave are outstanding (loads complete in
// issue order, so every older one has landed).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// ---- LoRA side path (app/gpu/ops.js:70-87: y = W x + sum_i s_i B_i (A_i x)) ----------------
// The LoRA term of one 32x32 output tile in the v_mfma_f32_32x32x16_f16 accumulator layout:
// D[m][n] = sum_k t[m][k] lb[n][k] over k < R (R % 32 == 0), with t fp32 [M][R] (the
// down-projected input, rounded to fp16 here) and lb fp16 [N][R] (the stacked up-projections).
// Lane l supplies row `mrow` of t and row `nrow` of lb (rows l % 32 of the tile, clamped into
// the matrices), k = 16s + 8(l/32) .. +7. The GEMM epilogues add D after the bias, where the
// reference adds its delta (gemm.js:159-162), one tile at a time so that it costs 16 registers
// beyond the accumulators. Each 32-wide chunk of R issues its loads before its two products.
__device__ __forceinline__ float16_t lora_tile(const float* __restrict__ t, const half_t* __restrict__ lb, int R,
                                               int mrow, int nrow, int hi) {
  const float* tp = t + (long long)mrow * R + 8 * hi;
  const half_t* bp = lb + (long long)nrow * R + 8 * hi;
  float16_t d;
#pragma unroll
  for (int r = 0; r < 16; ++r) d[r] = 0.f;
  for (int k0 = 0; k0 < R; k0 += 32) {
    const float4 x0 = *reinterpret_cast<const float4*>(tp + k0);
    const float4 x1 = *reinterpret_cast<const float4*>(tp + k0 + 4);
    const float4 y0 = *reinterpret_cast<const float4*>(tp + k0 + 16);
    const float4 y1 = *reinterpret_cast<const float4*>(tp + k0 + 20);
    const half8_t b0 = *reinterpret_cast<const half8_t*>(bp + k0);
    const half8_t b1 = *reinterpret_cast<const half8_t*>(bp + k0 + 16);
    const half8_t a0 = {(half_t)x0.x, (half_t)x0.y, (half_t)x0.z, (half_t)x0.w,
                        (half_t)x1.x, (half_t)x1.y, (half_t)x1.z, (half_t)x1.w};
    const half8_t a1 = {(half_t)y0.x, (half_t)y0.y, (half_t)y0.z, (half_t)y0.w,
                        (half_t)y1.x, (half_t)y1.y, (half_t)y1.z, (half_t)y1.w};
    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, d, 0, 0, 0);
    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, d, 0, 0, 0);
  }
  return d;
}

// The LoRA term of one output element by scalar products (GEMV and split-K reduce paths).
__device__ __forceinline__ float lora_dot(const float* __restrict__ t, const half_t* __restrict__ lb, int R,
                                          int m, int n) {
  const float* tp = t + (long long)m * R;
  const half_t* bp = lb + (long long)n * R;
  float d = 0.f;
  for (int k = 0; k < R; ++k) d += tp[k] * (float)bp[k];
  return d;
}

}  // namespace ns2dev
