// Joint image+text flash attention on MFMA (fp16 operands, fp32 accumulation).
//
// Two kernels per call:
//  1. pack: reads the fp32 q/k/v views, applies the optional per-head RMSNorm and split-half
//     RoPE (the DiT's headNorm, kernels.js:307-342), folds scale*log2(e) into q, and writes
//     head-major fp16 operands: Qp [B*H][Lq_pad][D], Kp [B*H][Lk_pad][D], Vt [B*H][D][Lk_pad]
//     (V transposed), plus one fp32 bias per key in log2 units (0 on image keys, the
//     log-prompt-weight on text keys, -1e30 on padding keys).
//  2. flash: one workgroup per (query block, head, batch); K/V tiles of 64 keys are staged in
//     LDS (double-buffered, register prefetch). Each wave owns QT x 32 queries and works in
//     the transposed domain so no register shuffles are needed between the two products:
//        S^T = K Q^T       (A = K rows from LDS, B = Q^T held in registers)
//        O^T += V^T P^T    (A = V^T rows from LDS, B = P^T straight from the S^T registers)
//     The 32x32 MFMA accumulator of S^T gives every lane one query column and 16 keys, which
//     is exactly the k-slice a lane supplies as B operand of the next product (the k order
//     inside an MFMA is free as long as A and B agree), and the online-softmax statistics
//     of a query live in the same lanes as its output column.
#include "ns2_common.h"

using namespace ns2dev;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaskBias = -1.0e30f;
constexpr int KB = 64;          // keys per tile
constexpr int QPAD = 256;       // Lq padding granule (largest query block)
constexpr int KPAD_LDS = 8;     // halfs of padding per LDS row

struct PackArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* key_bias;
  const float* q_norm;
  const float* k_norm;
  const float* cs;
  half_t* Qp;
  half_t* Kp;
  half_t* Vt;
  float* bias2;
  long long qOff, kOff, vOff, qBatch, kBatch, vBatch, biasBatch, sinOff;
  int Lq, Lk, Lq_pad, Lk_pad, H, ldq, ldk, ldv, biasStart, rope_rows;
  float qscale, eps;
};

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

// grid: (rows / 64, H, batch), 256 threads: 64 rows x 4 parts.
template <int D>
__global__ __launch_bounds__(256) void attn_pack_kernel(PackArgs a) {
  __shared__ half_t vs[D][KB + 2];
  const int h = blockIdx.y, b = blockIdx.z;
  const int bh = b * a.H + h;
  const int row0 = blockIdx.x * KB;
  const int tid = threadIdx.x;
  const int rl = tid >> 2, part = tid & 3;
  const int row = row0 + rl;

  // Q rows
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
  if (row0 < a.Lk_pad) {
    // K rows
    half_t* dst = a.Kp + ((long long)bh * a.Lk_pad + row) * D;
    if (row < a.Lk) {
      const float* src = a.k + a.kOff + b * a.kBatch + (long long)row * a.ldk + (long long)h * D;
      prep_row<D>(src, a.k_norm, a.cs, a.sinOff, row, a.cs && row < a.rope_rows, 1.0f, a.eps, part, dst);
    } else {
#pragma unroll
      for (int j = 0; j < D / 4; ++j) dst[part * (D / 4) + j] = (half_t)0.f;
    }
    // V rows -> transposed through LDS
    {
      const float* src = a.v + a.vOff + b * a.vBatch + (long long)row * a.ldv + (long long)h * D;
#pragma unroll
      for (int j = 0; j < D / 4; ++j) {
        const int d = part * (D / 4) + j;
        vs[d][rl] = (half_t)(row < a.Lk ? src[d] : 0.f);
      }
    }
    __syncthreads();
    for (int e = tid; e < D * KB; e += 256) {
      const int d = e / KB, kk = e % KB;
      a.Vt[((long long)bh * D + d) * a.Lk_pad + row0 + kk] = vs[d][kk];
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
}

struct FlashArgs {
  const half_t* Qp;
  const half_t* Kp;
  const half_t* Vt;
  const float* bias2;
  float* O;
  long long oOff, oBatch;
  int Lq, Lk, Lq_pad, Lk_pad, H, ldo;
  int bias_block0;  // first key tile that needs the per-key bias (text or padding keys)
};

template <int D, int QT, int NW>
__global__ __launch_bounds__(NW * 64) void flash_kernel(FlashArgs a) {
  constexpr int NT = NW * 64;
  constexpr int KROW = D + KPAD_LDS;    // K tile row (halfs)
  constexpr int VROW = KB + KPAD_LDS;   // V^T tile row (halfs)
  constexpr int DC = D / 16;            // k-steps of S
  constexpr int DT = D / 32;            // dim tiles of O
  constexpr int K_CHUNKS = KB * D / 8;  // 16-byte chunks per K tile
  constexpr int V_CHUNKS = D * KB / 8;
  constexpr int KC_T = (K_CHUNKS + NT - 1) / NT;
  constexpr int VC_T = (V_CHUNKS + NT - 1) / NT;

  __shared__ __attribute__((aligned(16))) half_t ks[2][KB * KROW];
  __shared__ __attribute__((aligned(16))) half_t vts[2][D * VROW];
  __shared__ float kbias[2][KB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y, b = blockIdx.z, bh = b * a.H + h;
  const int q0 = blockIdx.x * (NW * QT * 32) + wave * QT * 32;
  const int lq = lane & 31, hi = lane >> 5;

  const half_t* Kg = a.Kp + (long long)bh * a.Lk_pad * D;
  const half_t* Vg = a.Vt + (long long)bh * D * a.Lk_pad;
  const float* Bg = a.bias2 + (long long)b * a.Lk_pad;

  // Q^T operands: lane holds query q0 + qt*32 + lq, dims c*16 + 8*hi .. +7
  half8_t qf[QT][DC];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const half_t* qrow = a.Qp + ((long long)bh * a.Lq_pad + q0 + qt * 32 + lq) * D + 8 * hi;
#pragma unroll
    for (int c = 0; c < DC; ++c) qf[qt][c] = *reinterpret_cast<const half8_t*>(qrow + c * 16);
  }

  float16_t o[QT][DT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qt][dt][r] = 0.f;
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = kMaskBias;
    l_run[qt] = 0.f;
  }

  uint4 kreg[KC_T], vreg[VC_T];
  float breg = 0.f;
  auto gload = [&](int t) {
    const int key0 = t * KB;
#pragma unroll
    for (int i = 0; i < KC_T; ++i) {
      const int c = tid + i * NT;
      if (c < K_CHUNKS) kreg[i] = *reinterpret_cast<const uint4*>(Kg + (long long)key0 * D + c * 8);
    }
#pragma unroll
    for (int i = 0; i < VC_T; ++i) {
      const int c = tid + i * NT;
      if (c < V_CHUNKS) {
        const int d = c / (KB / 8), kc = (c % (KB / 8)) * 8;
        vreg[i] = *reinterpret_cast<const uint4*>(Vg + (long long)d * a.Lk_pad + key0 + kc);
      }
    }
    if (tid < KB) breg = Bg[key0 + tid];
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KC_T; ++i) {
      const int c = tid + i * NT;
      if (c < K_CHUNKS) {
        const int key = c / (D / 8), dc = (c % (D / 8)) * 8;
        *reinterpret_cast<uint4*>(&ks[buf][key * KROW + dc]) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VC_T; ++i) {
      const int c = tid + i * NT;
      if (c < V_CHUNKS) {
        const int d = c / (KB / 8), kc = (c % (KB / 8)) * 8;
        *reinterpret_cast<uint4*>(&vts[buf][d * VROW + kc]) = vreg[i];
      }
    }
    if (tid < KB) kbias[buf][tid] = breg;
  };

  const int ntiles = a.Lk_pad / KB;
  gload(0);
  sstore(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1;
    if (t + 1 < ntiles) gload(t + 1);

    // ---- S^T = K Q^T: s[kt][qt][r] = score(key t*64 + kt*32 + 8(r/4) + 4hi + r%4, query lq)
    float16_t s[2][QT];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kt][qt][r] = 0.f;
      const half_t* krow = &ks[cur][(kt * 32 + lq) * KROW + 8 * hi];
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const half8_t kf = *reinterpret_cast<const half8_t*>(krow + c * 16);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          s[kt][qt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[qt][c], s[kt][qt], 0, 0, 0);
      }
    }

    // ---- per-key bias (text keys and padding keys only)
    if (t >= a.bias_block0) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 bb = *reinterpret_cast<const float4*>(&kbias[cur][kt * 32 + 8 * g + 4 * hi]);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            s[kt][qt][4 * g + 0] += bb.x;
            s[kt][qt][4 * g + 1] += bb.y;
            s[kt][qt][4 * g + 2] += bb.z;
            s[kt][qt][4 * g + 3] += bb.w;
          }
        }
    }

    // ---- online softmax (log2 domain) and P^T operands
    half8_t pf[QT][2][2];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = s[0][qt][0];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kt][qt][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[qt], mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
      m_run[qt] = m_new;
      float ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pv = __builtin_amdgcn_exp2f(s[kt][qt][kk * 8 + e] - m_new);
            const half_t ph = (half_t)pv;
            pf[qt][kt][kk][e] = ph;
            ls += (float)ph;
          }
      l_run[qt] = l_run[qt] * alpha + ls;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[qt][dt][r] *= alpha;
    }

    // ---- O^T += V^T P^T: A = V^T[dim dt*32 + lq][keys kt*32 + kk*16 + {4hi..4hi+3, 8+4hi..}]
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const half_t* vrow = &vts[cur][(dt * 32 + lq) * VROW + 4 * hi];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const half4_t v0 = *reinterpret_cast<const half4_t*>(vrow + kt * 32 + kk * 16);
          const half4_t v1 = *reinterpret_cast<const half4_t*>(vrow + kt * 32 + kk * 16 + 8);
          const half8_t vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
          for (int qt = 0; qt < QT; ++qt)
            o[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[qt][kt][kk], o[qt][dt], 0, 0, 0);
        }
    }

    if (t + 1 < ntiles) sstore(cur ^ 1);
    __syncthreads();
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

template <int D>
int run_attention(PackArgs pa, FlashArgs fa, int batch) {
  hipStream_t s = ns2::stream();
  const int rows = pa.Lq_pad > pa.Lk_pad ? pa.Lq_pad : pa.Lk_pad;
  {
    ns2::ProfScope prof_("attn_pack");
    attn_pack_kernel<D><<<dim3(rows / KB, pa.H, batch), 256, 0, s>>>(pa);
    NS2_LAUNCHED("attn_pack");
  }
  ns2::ProfScope prof_("attn_flash");
  // 2 query tiles of 32 per wave; 4 waves per workgroup when that still gives every CU
  // a workgroup, else 2.
  const long long units4 = (long long)((pa.Lq + 255) / 256) * pa.H * batch;
  if (units4 >= 256) {
    dim3 grid((pa.Lq + 255) / 256, pa.H, batch);
    flash_kernel<D, 2, 4><<<grid, 256, 0, s>>>(fa);
  } else {
    dim3 grid((pa.Lq + 127) / 128, pa.H, batch);
    flash_kernel<D, 2, 2><<<grid, 128, 0, s>>>(fa);
  }
  NS2_LAUNCHED("attn_flash");
  return NS2_OK;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int ns2_attention(const float* q, const float* k, const float* v, float* o, int batch,
                             int Lq, int Lk, int H, int D, int ldq, int ldk, int ldv, int ldo,
                             long long qOff, long long kOff, long long vOff, long long oOff,
                             long long qBatch, long long kBatch, long long vBatch, long long oBatch,
                             float scale, const float* key_bias, int biasStart, long long biasBatch,
                             const float* q_norm, const float* k_norm, float eps,
                             const float* rope_cs, long long sin_off, int rope_rows) {
  NS2_READY();
  if (Lq <= 0 || batch <= 0) return NS2_OK;
  NS2_REQUIRE(q && k && v && o, "ns2_attention: null q, k, v or o");
  NS2_REQUIRE(D == 32 || D == 64 || D == 96 || D == 128, "ns2_attention: unsupported head dim %d", D);
  NS2_REQUIRE(Lk > 0 && H > 0, "ns2_attention: Lk=%d H=%d", Lk, H);
  NS2_REQUIRE(ldo % 4 == 0 && oOff % 4 == 0 && oBatch % 4 == 0 && aligned16(o),
              "ns2_attention: the output view must be 16-byte aligned (ldo, oOff, oBatch multiples of 4)");
  NS2_REQUIRE(ldq >= H * D || qOff > 0 || ldq >= D, "ns2_attention: bad ldq");
  const int Lq_pad = (Lq + QPAD - 1) / QPAD * QPAD;
  const int Lk_pad = (Lk + KB - 1) / KB * KB;
  const long long bh = (long long)batch * H;
  const size_t qbytes = (size_t)bh * Lq_pad * D * sizeof(half_t);
  const size_t kbytes = (size_t)bh * Lk_pad * D * sizeof(half_t);
  const size_t bbytes = (size_t)batch * Lk_pad * sizeof(float);
  half_t* Qp = static_cast<half_t*>(ns2::workspace(1, qbytes));
  half_t* Kp = static_cast<half_t*>(ns2::workspace(2, kbytes));
  half_t* Vt = static_cast<half_t*>(ns2::workspace(3, kbytes));
  float* B2 = static_cast<float*>(ns2::workspace(4, bbytes));
  if (!Qp || !Kp || !Vt || !B2) return ns2::set_error(NS2_ERR_OOM, "ns2_attention: workspace allocation failed");

  PackArgs pa{q, k, v, key_bias, q_norm, k_norm, rope_cs, Qp, Kp, Vt, B2,
              qOff, kOff, vOff, qBatch, kBatch, vBatch, biasBatch, sin_off,
              Lq, Lk, Lq_pad, Lk_pad, H, ldq, ldk, ldv, biasStart, rope_rows,
              scale * kLog2e, eps};
  int first_biased = Lk;  // padding keys need the mask bias too
  if (key_bias && biasStart < Lk) first_biased = biasStart < 0 ? 0 : biasStart;
  FlashArgs fa{Qp, Kp, Vt, B2, o, oOff, oBatch, Lq, Lk, Lq_pad, Lk_pad, H, ldo, first_biased / KB};
  if (key_bias) NS2_REQUIRE(biasStart >= 0, "ns2_attention: negative biasStart");
  switch (D) {
    case 32: return run_attention<32>(pa, fa, batch);
    case 64: return run_attention<64>(pa, fa, batch);
    case 96: return run_attention<96>(pa, fa, batch);
    default: return run_attention<128>(pa, fa, batch);
  }
}
