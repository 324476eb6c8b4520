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
constexpr int kWorkspaceSlots = 6;

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

// Sum over the 64 lanes of a wave.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// One radix-4 stage of the regular Hadamard H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]
// across 4 lanes whose lane bits (lo, lo<<1) index the 4 inputs: output position i is
// (a+b+c+e) - 2 * input[3 - i], and position 3 - i is lane ^ (3 * lo).
__device__ __forceinline__ float h4_lanes(float v, int lo) {
  float s = v + __shfl_xor(v, lo, 64);
  s += __shfl_xor(s, 2 * lo, 64);
  float partner = __shfl_xor(v, 3 * lo, 64);
  return s - 2.0f * partner;
}

// In-wave fast Walsh-Hadamard transform of one 256-group: lane t holds elements 4t..4t+3
// in v[0..3]. Computes y = x H with H = kron(H4, H4, H4, H4) / 16 (tools/quant.py:21-29):
// radix-4 stages at strides 1 (in registers), 4, 16 and 64 (across lanes).
__device__ __forceinline__ void fwht256_wave(float v[4]) {
  {
    float a = v[0], b = v[1], c = v[2], e = v[3];
    float s = a + b + c + e;
    v[0] = s - 2.0f * e;
    v[1] = s - 2.0f * c;
    v[2] = s - 2.0f * b;
    v[3] = s - 2.0f * a;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = h4_lanes(v[j], 1);   // stride 4: lane bits 0-1
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = h4_lanes(v[j], 4);   // stride 16: lane bits 2-3
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = h4_lanes(v[j], 16);  // stride 64: lane bits 4-5
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] *= 0.0625f;
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

}  // namespace ns2dev
