/*
 * ns2.h -- C ABI of the MI355X (gfx950) kernel library for one Nanosaur2 DiT pass.
 *
 * This library replaces the WebGPU runtime and the WGSL kernels behind the reference's
 * ops layer (app/gpu/device.js, app/gpu/ops.js, app/gpu/kernels.js, app/gpu/gemm.js).
 * A Node.js N-API addon (nanosaur2-web_amd/addon/ns2_addon.cc) exposes exactly these
 * entry points to the JavaScript host; Python binds them through ctypes.
 *
 * Conventions
 *  - Every entry point returns an int status: NS2_OK (0) or an error code; the message of
 *    the last error on the calling thread is returned by ns2_last_error().
 *  - Pointers named like tensors are DEVICE pointers (from ns2_malloc / ns2_pool_get, or
 *    any other HIP device allocation). Host pointers are only taken by ns2_h2d / ns2_d2h.
 *  - Activations are fp32, row-major. Strides (ld*) and offsets (*Off) are in ELEMENTS,
 *    exactly as in the reference's dispatch parameters.
 *  - All launches are asynchronous and ordered on one HIP stream (ns2_set_stream; the
 *    default is a stream the library creates at ns2_init, default priority). ns2_sync /
 *    ns2_d2h wait for completion.
 *  - int8 weights are "int8_tensorwise + convrot": W_q int8 [N, K] row-major with one fp32
 *    scale per output row; the layer computes (x H) W_q^T diag(scale), where H is the
 *    normalized 256-point regular Hadamard matrix applied per 256-feature group
 *    (tools/quant.py:21-64).
 *  - bf16 weights are raw bfloat16 bit patterns [N, K] row-major (uint16_t).
 */
#ifndef NS2_H
#define NS2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------ */
#define NS2_OK 0
#define NS2_ERR_INVALID 1 /* bad argument or unsupported shape/alignment */
#define NS2_ERR_HIP 2     /* HIP runtime / launch error */
#define NS2_ERR_OOM 3     /* device allocation failed */
#define NS2_ERR_STATE 4   /* library not initialised */

/* activation codes (gemm.js:163, kernels.js:9-17) */
#define NS2_ACT_NONE 0
#define NS2_ACT_SILU 1
#define NS2_ACT_GELU_TANH 2

/* elementwise op codes (kernels.js:496-518) */
#define NS2_EW_ADD 0
#define NS2_EW_SUB 1
#define NS2_EW_SILU 2
#define NS2_EW_COPY 3

/* ---- runtime: replaces GPU / BufferPool / Profiler of app/gpu/device.js -------------- */

/* GPU.create (app/gpu/device.js:61-81): select and initialise a device. */
int ns2_init(int device);
/* Message of the last failed call on this thread ("" if none). */
const char* ns2_last_error(void);
/* gpu.info (app/gpu/device.js:77): device name, compute units, HBM bytes. */
int ns2_device_info(char* name, size_t cap, int* compute_units, size_t* hbm_bytes);
/* Use a caller-owned hipStream_t for every later launch (NULL = null stream). */
int ns2_set_stream(void* hip_stream);
void* ns2_get_stream(void);

/* GPU.upload (app/gpu/device.js:134-139): persistent (non-pooled) device buffer. */
int ns2_malloc(void** ptr, size_t bytes);
int ns2_free(void* ptr);
/* BufferPool.round (app/gpu/device.js:33-39): 1/8-power-of-two size buckets, >= 256 B. */
size_t ns2_pool_round(size_t bytes);
/* BufferPool.get (app/gpu/device.js:40-48); *rounded receives the bucket size. */
int ns2_pool_get(size_t bytes, void** ptr, size_t* rounded);
/* BufferPool.put / Tensor.release (app/gpu/device.js:20-23, 49-52). */
int ns2_pool_put(void* ptr, size_t rounded);
/* BufferPool.trim (app/gpu/device.js:53-56). */
int ns2_pool_trim(void);
/* BufferPool.allocated / .peak (app/gpu/device.js:30-31). */
int ns2_pool_stats(size_t* allocated, size_t* peak);

/* GPU.write (app/gpu/device.js:122-131): host -> device, ordered on the stream; src may be
 * reused when this returns. Copies up to 64 KB go through pinned staging slots and do not wait
 * for the work queued before them (the queued write of the reference's writeBuffer); larger ones
 * wait for the stream. Refused inside a graph capture. */
int ns2_h2d(void* dst, const void* src, size_t bytes);
/* GPU.read (app/gpu/device.js:141-154): device -> host, waits for prior work. */
int ns2_d2h(void* dst, const void* src, size_t bytes);
/* GPU.sync (app/gpu/device.js:218-222): wait for all queued work, surface errors. */
int ns2_sync(void);
/* Fill count 32-bit words with value (a kernel, safe inside graph capture).
 * ops.zero (app/gpu/ops.js:89-93) is value = 0. */
int ns2_fill_u32(void* dst, uint32_t value, size_t count);

/* Recorded launch sequences (HIP graphs), the analogue of the reference's command-buffer
 * batching (app/gpu/device.js:196-215: dispatches recorded into one encoder, submitted on
 * flush). Launches issued between ns2_graph_begin and ns2_graph_end are recorded, not run;
 * ns2_graph_launch replays them on the stream with the same buffer addresses. No call inside
 * a capture may wait for the stream (ns2_h2d, ns2_d2h, ns2_sync fail and void the capture), and
 * the recorded launches should have run eagerly once with the same shapes, so that no
 * workspace grows during the capture. While a graph is alive, ns2_pool_trim frees nothing and
 * replaced workspace buffers are kept until the last ns2_graph_destroy. */
int ns2_graph_begin(void);
int ns2_graph_end(void** graph);
int ns2_graph_launch(void* graph);
int ns2_graph_destroy(void* graph);

/* Profiler (app/gpu/device.js:234-288): stream-ordered timing events. */
int ns2_event_create(void** ev);
int ns2_event_record(void* ev);
int ns2_event_elapsed(void* start, void* end, float* ms);
int ns2_event_destroy(void* ev);
/* Kernel-level Profiler: while enabled, stream events bracket every kernel launch of the
 * library; ns2_profile_report writes JSON {"<kernel>": {"count": n, "ms": total}, ...} with
 * the sums since the last ns2_profile_reset (waits for the recorded events). */
int ns2_profile_enable(int on);
int ns2_profile_reset(void);
int ns2_profile_report(char* buf, size_t cap);

/* ---- ConvRot rotation --------------------------------------------------------------- */

/* ops.rotate + hadamardShader (app/gpu/ops.js:38-44, app/gpu/kernels.js:378-407):
 * y = x H per contiguous group of 256 fp32 values, groups = size / 256. y may equal x. */
int ns2_hadamard256(const float* x, float* y, long long groups);
/* Same rotation on a strided [rows, cols] view (cols % 256 == 0), written as fp16: the
 * pre-rotated operand of the int8 linear. tiled == 0: row-major with ldy (fp16 elements), the
 * `xr` of ns2_linear_i8; tiled != 0: the tiled layout of ns2_linear_i8_tiled (ldy ignored;
 * y holds ceil(rows/64)*64 rows). */
int ns2_rotate_f16(const float* x, int ldx, uint16_t* y, int ldy, int rows, int cols, int tiled);

/* ---- linear layers (ops.linear, app/gpu/ops.js:50-66; runMatmul :14-32;
 *      matmulShader epilogue app/gpu/gemm.js:159-164) -------------------------------------
 * C[cOff + m*ldc + n] (=|+=) epilogue(alpha * sum_k A[m,k] W[n,k]) for m < M, n < N with
 *   r = acc*alpha; r *= scale[n] (int8 only); r += bias[n]; r += add[m*N + n]; r = act(r);
 *   resid == 0: C = r;  resid != 0 && gate == NULL: C += r;  else C += gate[gOff + n] * r.
 * bias, add and gate may be NULL. */

/* int8 ConvRot weights. a_fmt selects the activation operand:
 *   a_fmt = 0: A is fp32 [M, lda], NOT rotated; the call rotates it (ops.linear without xr).
 *   a_fmt = 1: A is fp16 [M, lda] already rotated (the fused producers' output).
 *   a_fmt = 2: A is fp32 [M, lda] already rotated (ops.linear with opts.xr = ops.rotate(x)).
 * Requires K % 256 == 0. */
int ns2_linear_i8(const void* A, int a_fmt, int lda, const int8_t* W, const float* scale,
                  const float* bias, const float* add, float* C, int M, int N, int K, int ldc,
                  long long cOff, float alpha, int act, int resid, const float* gate,
                  long long gOff);
/* The same int8 ConvRot linear on tiled operands (the fused DiT path): At is the rotated
 * fp16 activation in the tiled layout [ceil(M/64)][K/64][8][64][8] written by the fused
 * producers (tiled != 0), Wt the weight re-tiled by ns2_tile_i8_weight. Epilogue as above
 * without `add`. Requires N % 64 == 0, K % 256 == 0. */
int ns2_linear_i8_tiled(const uint16_t* At, const int8_t* Wt, const float* scale,
                        const float* bias, float* C, int M, int N, int K, int ldc,
                        long long cOff, float alpha, int act, int resid, const float* gate,
                        long long gOff);
/* Re-tile an int8 weight [N, K] row-major into Wt [N/64][K/64][8][64][8 bytes] for
 * ns2_linear_i8_tiled, each byte stored biased as w + 128 (N % 64 == 0, K % 64 == 0).
 * Done once when the weight is loaded. */
int ns2_tile_i8_weight(const int8_t* W, int8_t* Wt, int N, int K);
/* The GLU MLP's first linear fused with the GLU and the rotation of its output (fused DiT
 * path): with h = (At Wt^T) * alpha * scale + bias (N = 2I columns), writes
 * Y = rotate(act(h[:, :I]) * h[:, I:]) as the tiled fp16 operand of the next int8 linear
 * (ceil(M/64)*64 rows of I columns). Replaces ops.linear (app/gpu/ops.js:46-66) + ops.glu
 * (ops.js:140-148) + ops.rotate (ops.js:37-44) on the MLP path (app/models/nanosaur2.js:142-152).
 * Wt must come from ns2_tile_i8_weight_glu. N % 512 == 0, K % 256 == 0. */
int ns2_linear_i8_glu_rot_tiled(const uint16_t* At, const int8_t* Wt, const float* scale,
                                const float* bias, uint16_t* Y, int M, int N, int K, float alpha,
                                int act);
/* ns2_tile_i8_weight for ns2_linear_i8_glu_rot_tiled: tiled row 64q + t holds weight row
 * 32q + t (t < 32) or N/2 + 32q + t - 32 (t >= 32), pairing the two GLU halves. */
int ns2_tile_i8_weight_glu(const int8_t* W, int8_t* Wt, int N, int K);
/* bf16 weights (gemm.js:98-118), fp32 activations [M, lda]. Requires K % 16 == 0. */
int ns2_linear_bf16(const float* A, int lda, const uint16_t* W, const float* bias,
                    const float* add, float* C, int M, int N, int K, int ldc, long long cOff,
                    float alpha, int act, int resid, const float* gate, long long gOff);
/* The bf16 linear of ns2_linear_bf16 (gemm.js:98-118, ops.linear app/gpu/ops.js:46-66) on tiled
 * operands, for many rows (the DiT's 3952-row patch embedder, SPRINT projection and final
 * layer): At is the fp16 activation in the tiled layout of ns2_linear_i8_tiled (written by
 * ns2_to_tiled_f16 or ns2_norm_mod_f16), Wt the weight re-tiled as fp16 by
 * ns2_tile_bf16_weight. Epilogue as above without `add` (no row scale). N % 64 == 0,
 * K % 64 == 0. The operands are the fp16 values the row-major kernel's loaders convert its
 * fp32 activations and bf16 weights to. Additive to the reference interface. */
int ns2_linear_f16w_tiled(const uint16_t* At, const uint16_t* Wt, const float* bias, float* C, int M, int N, int K,
                          int ldc, long long cOff, float alpha, int act, int resid, const float* gate,
                          long long gOff);
/* Re-tile a bf16 weight [N, K] row-major into fp16 tiles Wt [N/64][K/64][8][64][8 halfs] for
 * ns2_linear_f16w_tiled (round to nearest even; N % 64 == 0, K % 64 == 0). Done once at load. */
int ns2_tile_bf16_weight(const uint16_t* W, uint16_t* Wt, int N, int K);

/* ---- LoRA side path (ops.linear with W.lora, app/gpu/ops.js:50-87 loraDelta; app/lora.js) ---
 * The _lora variants compute the same linear plus the low-rank term
 *   r += sum_k t[m,k] lora_b[n,k],  t = x lora_a^T,
 * added after the bias, where the reference adds its `delta` (ADD, gemm.js:162), so it is not
 * scaled by alpha or the int8 row scale. x is the linear's GEMM input: the rotated operand for
 * int8 weights (so lora_a holds the down-projections rotated per 256-group, app/lora.js:61-78),
 * the fp32 activations for bf16 weights.
 *   lora_a: fp16 [lora_r, K], the down-projections A_i of every LoRA on the weight, stacked;
 *   lora_b: fp16 [N, lora_r], column block i = strength_i * alpha_i / r_i * B_i in the rows of
 *           its output window [off_i, off_i + n_i) and zero elsewhere (app/lora.js:144-152);
 *   lora_r: the stacked rank, a multiple of 32 (pad with zero rows/columns), at most 256.
 * Both 16-byte aligned; lora_b in the weight's original row order (also for the GLU-interleaved
 * tiles of ns2_linear_i8_glu_rot_tiled). lora_r = 0 is the plain entry point. t lives in
 * library scratch. Additive to the reference interface (its loraDelta materializes the
 * [M, N] delta; here the term starts the GEMM accumulators). */
int ns2_linear_i8_lora(const void* A, int a_fmt, int lda, const int8_t* W, const float* scale,
                       const float* bias, const float* add, float* C, int M, int N, int K, int ldc,
                       long long cOff, float alpha, int act, int resid, const float* gate,
                       long long gOff, const uint16_t* lora_a, const uint16_t* lora_b, int lora_r);
int ns2_linear_i8_tiled_lora(const uint16_t* At, const int8_t* Wt, const float* scale,
                             const float* bias, float* C, int M, int N, int K, int ldc,
                             long long cOff, float alpha, int act, int resid, const float* gate,
                             long long gOff, const uint16_t* lora_a, const uint16_t* lora_b, int lora_r);
int ns2_linear_i8_glu_rot_tiled_lora(const uint16_t* At, const int8_t* Wt, const float* scale,
                                     const float* bias, uint16_t* Y, int M, int N, int K, float alpha,
                                     int act, const uint16_t* lora_a, const uint16_t* lora_b, int lora_r);
int ns2_linear_bf16_lora(const float* A, int lda, const uint16_t* W, const float* bias,
                         const float* add, float* C, int M, int N, int K, int ldc, long long cOff,
                         float alpha, int act, int resid, const float* gate, long long gOff,
                         const uint16_t* lora_a, const uint16_t* lora_b, int lora_r);
int ns2_linear_f16w_tiled_lora(const uint16_t* At, const uint16_t* Wt, const float* bias, float* C, int M, int N,
                               int K, int ldc, long long cOff, float alpha, int act, int resid, const float* gate,
                               long long gOff, const uint16_t* lora_a, const uint16_t* lora_b, int lora_r);

/* ---- attention without the fused kernel (ops.attention's materialized path, app/gpu/ops.js:
 *      211-241, softmaxShader) -----------------------------------------------------------
 * For heads h < H with K/V head g = h / group:
 *   s_ij = <q_i, k_j> / sqrt(D), masked to j <= i when causal;
 *   O[i*ldo + h*D ..] = sum_j softmax_j(s_ij) v_j,
 * q_i = Q[qOff + i*ldq + h*D ..], k_j = K[kOff + j*ldk + g*D ..], v_j = V[vOff + j*ldv + g*D ..].
 * fp32 throughout. D <= 256, H % group == 0; no key bias (the reference rejects a bias on this
 * path). Used for causal / grouped-head attention (the Gemma3 text encoder). */
int ns2_attention_rows(const float* q, const float* k, const float* v, float* o, int Lq, int Lk,
                       int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff,
                       long long kOff, long long vOff, int group, int causal);
/* ns2_attention_rows with K and V stored as fp16 (ldk, ldv, kOff, vOff counted in fp16
 * elements), as ns2_linear_bf16_head_norm_f16kv writes them. The products take fp16 operands on
 * either entry, so for K/V that are the fp16 roundings of ns2_attention_rows' fp32 K/V the
 * outputs are the same bit for bit. D a multiple of 16 up to 256; q rows and the K/V rows
 * 16-byte aligned. Additive to the reference interface. */
int ns2_attention_rows_f16kv(const float* q, const uint16_t* k, const uint16_t* v, float* o, int Lq, int Lk,
                             int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff,
                             long long kOff, long long vOff, int group, int causal);
/* ns2_attention_rows_f16kv followed by the sublayer's output projection split over heads
 * (Gemma3's attention and o_proj, app/models/gemma3.js:67-73): for each head h, with O_h its attention output
 * [Lq, D] rounded to fp16 (as a linear rounds its input), part[h] [Lq, N] = O_h W_o[:, hD:(h+1)D]^T,
 * fp32. wo_tiled: W_o [N, H*D] as ns2_tile_bf16_weight writes it. The H shares sum to the
 * projection (without bias); ns2_parts_add_rmsnorm adds them. N and H*D multiples of 64.
 * Additive to the reference interface. */
int ns2_attention_rows_f16kv_oproj(const float* q, const uint16_t* k, const uint16_t* v, const uint16_t* wo_tiled,
                                   float* part, int Lq, int Lk, int H, int D, int ldq, int ldk, int ldv,
                                   long long qOff, long long kOff, long long vOff, int group, int causal, int N);

/* ---- attention (ops.attention, app/gpu/ops.js:199-209; flashAttentionShader,
 *      app/gpu/kernels.js:119-305) ----------------------------------------------------------
 * For every batch element b and head h < H, with q_i = Q[qOff + b*qBatch + i*ldq + h*D ..],
 * k_j, v_j likewise and
 *   s_ij = scale * <q_i, k_j> + (j >= biasStart ? key_bias[b*biasBatch + j - biasStart] : 0)
 *   O[oOff + b*oBatch + i*ldo + h*D ..] = sum_j softmax_j(s_ij) v_j      (non-causal, group 1)
 * Optional fused prologue, applied to the operands before the product (the work the DiT
 * does with headNorm, app/gpu/kernels.js:307-342, app/models/nanosaur2.js:199-204):
 *   q_norm / k_norm: per-head RMSNorm x * rsqrt(mean x^2 + eps) * w[D] on every q / k row;
 *   rope_cs: split-half RoPE (pair i, i + D/2) on q rows and k rows with index < rope_rows,
 *            cos at rope_cs[row*D/2 + i], sin at rope_cs[sin_off + row*D/2 + i].
 * key_bias may be NULL. D must be 32, 64, 96 or 128. */
int ns2_attention(const float* q, const float* k, const float* v, float* o, int batch,
                  int Lq, int Lk, int H, int D, int ldq, int ldk, int ldv, int ldo,
                  long long qOff, long long kOff, long long vOff, long long oOff,
                  long long qBatch, long long kBatch, long long vBatch, long long oBatch,
                  float scale, const float* key_bias, int biasStart, long long biasBatch,
                  const float* q_norm, const float* k_norm, float eps, const float* rope_cs,
                  long long sin_off, int rope_rows);

/* ns2_attention (batch 1) whose key and value rows from text_start on come from a second view:
 * key row r >= text_start is k_text[(r - text_start) * ld_text + h*D ..], value row likewise in
 * v_text; rows below text_start come from k / v as in ns2_attention. This is the DiT's joint
 * attention with the text keys projected apart from the image rows (app/models/nanosaur2.js:
 * 199-208: rows [L, L + T) of qkv hold the kv_y projection of the text; here the projections
 * of all joint blocks run as one GEMM and each block's attention reads its columns). k_norm
 * and the key bias apply to the text rows as to the others; RoPE only to rows < rope_rows. */
int ns2_attention_text(const float* q, const float* k, const float* v, float* o, int Lq, int Lk, int H, int D,
                       int ldq, int ldk, int ldv, int ldo, long long qOff, long long kOff, long long vOff,
                       long long oOff, float scale, const float* key_bias, int biasStart, const float* q_norm,
                       const float* k_norm, float eps, const float* rope_cs, long long sin_off, int rope_rows,
                       const float* k_text, const float* v_text, int ld_text, int text_start);

/* The q|k|v projection and the attention of one DiT block with the values handed over in the
 * attention's own fp16 layout instead of as fp32 rows (app/models/nanosaur2.js:193-208, the
 * `qkv` linear followed by ops.attention; app/gpu/ops.js:46-66 and :199-242). The two calls
 * give the same results as ns2_linear_i8_tiled + ns2_attention_text: the values are rounded
 * to fp16 once, in the GEMM epilogue instead of in the attention's operand pack.
 *
 * ns2_attention_vpack_bytes: size of the packed-value buffer vpk for Lk keys of H heads of D
 * (H * ceil(Lk/64)*64 * D halfs).
 *
 * ns2_linear_i8_tiled_vpack: ns2_linear_i8_tiled_lora (resid 0) whose output columns
 * [vcol0, vcol0 + H*D) -- the last H*D columns, vcol0 % 64 == 0, D % 32 == 0 -- are written to
 * vpk as the values of keys [0, M) of an attention over Lk >= M keys, instead of into C;
 * M % 16 == 0. Columns below vcol0 go to C as usual (their part of C is all that is written).
 *
 * ns2_attention_vpacked: ns2_attention_text (k_text/v_text may be null for a single view)
 * whose values of keys [0, v_rows) are taken from vpk as ns2_linear_i8_tiled_vpack wrote them;
 * the values of keys from v_rows on (text and padding keys) are packed into vpk from v / v_text
 * as usual. v_rows % 16 == 0, v_rows <= Lk; every view 16-byte aligned. */
size_t ns2_attention_vpack_bytes(int Lk, int H, int D);
int ns2_linear_i8_tiled_vpack(const uint16_t* At, const int8_t* Wt, const float* scale,
                              const float* bias, float* C, int M, int N, int K, int ldc,
                              long long cOff, float alpha, int act, const uint16_t* lora_a,
                              const uint16_t* lora_b, int lora_r, uint16_t* vpk, int vcol0, int H,
                              int D, int Lk);
int ns2_attention_vpacked(const float* q, const float* k, const float* v, float* o, int Lq, int Lk,
                          int H, int D, int ldq, int ldk, int ldv, int ldo, long long qOff,
                          long long kOff, long long vOff, long long oOff, float scale,
                          const float* key_bias, int biasStart, const float* q_norm,
                          const float* k_norm, float eps, const float* rope_cs, long long sin_off,
                          int rope_rows, const float* k_text, const float* v_text, int ld_text,
                          int text_start, uint16_t* vpk, int v_rows);

/* Bytes of the fixed device scratch array behind ns2_attention_noalloc (one per GPU, held
 * until the process ends). */
#define NS2_NOALLOC_SCRATCH_BYTES (64u << 20)

/* ns2_attention without any device allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments, semantics and results as
 * ns2_attention; its packed K/V tiles, key biases and (for views that are not 16-byte aligned)
 * packed queries live in a static device array of NS2_NOALLOC_SCRATCH_BYTES instead of
 * library workspace, and it calls no hipMalloc / hipFree. It needs
 *   2 * batch*H * ceil(Lk/64)*64 * D * 2  +  batch * ceil(Lk/64)*64 * 4
 *   (+ batch*H * ceil(Lq/256)*256 * D * 2 for unaligned views) bytes, each part rounded up to
 * 256, and fails with NS2_ERR_INVALID beyond the array: the 832x1216 joint attention
 * (3952 + 256 keys, 16 heads of 96) fits at batch 2. The array is shared by every call on a
 * GPU and keeps the last call's contents (every byte a call reads it writes first): calls that
 * overlap on one GPU (several streams or threads) race. */
int ns2_attention_noalloc(const float* q, const float* k, const float* v, float* o, int batch,
                          int Lq, int Lk, int H, int D, int ldq, int ldk, int ldv, int ldo,
                          long long qOff, long long kOff, long long vOff, long long oOff,
                          long long qBatch, long long kBatch, long long vBatch, long long oBatch,
                          float scale, const float* key_bias, int biasStart, long long biasBatch,
                          const float* q_norm, const float* k_norm, float eps, const float* rope_cs,
                          long long sin_off, int rope_rows);

/* ---- row kernels ---------------------------------------------------------------------- */

/* ops.headNorm + headNormShader (app/gpu/ops.js:133-138, app/gpu/kernels.js:307-342):
 * in place on X[(rowOff + l)*ld + colOff + h*D ..] for l < L, h < H; cs may be NULL. */
int ns2_head_norm(float* X, const float* w, int L, int H, int D, int ld, long long colOff,
                  long long rowOff, const float* cs, long long sinOff, float eps);
/* Two ops.headNorm calls on adjacent head ranges of the same rows in one launch: heads
 * [0, H1) with w1, then heads [H1, H1 + H2) with w2, from colOff on (Gemma3's q and k norms of
 * the packed q/k/v rows, app/models/gemma3.js:64-67). Additive to the reference interface. */
int ns2_head_norm2(float* X, const float* w1, int H1, const float* w2, int H2, int L, int D, int ld,
                   long long colOff, long long rowOff, const float* cs, long long sinOff, float eps);
/* ops.normMod + normModShader (app/gpu/ops.js:121-129, app/gpu/kernels.js:82-117):
 * y = norm(x) * (1 + mod[scaleOff + c]) + mod[shiftOff + c]; weight != NULL: RMSNorm * w,
 * weight == NULL: LayerNorm without affine. */
int ns2_norm_mod(const float* x, const float* mod, long long shiftOff, long long scaleOff,
                 int rows, int cols, const float* weight, float eps, float* y);
/* ns2_norm_mod followed by the ConvRot rotation, written as fp16 (cols % 256 == 0):
 * the pre-rotated input of the int8 linear that consumes it, row-major [rows, cols]
 * (tiled == 0) or in the layout of ns2_linear_i8_tiled (tiled != 0). */
int ns2_norm_mod_rotate_f16(const float* x, const float* mod, long long shiftOff,
                            long long scaleOff, int rows, int cols, const float* weight,
                            float eps, uint16_t* y, int tiled);
/* ns2_norm_mod without the rotation, written as fp16 (cols % 256 == 0, at most 4096): the
 * input of a tiled fp16-weight linear (the DiT's final layer, app/models/nanosaur2.js:252-253),
 * row-major or tiled as in ns2_norm_mod_rotate_f16. Additive to the reference interface. */
int ns2_norm_mod_f16(const float* x, const float* mod, long long shiftOff, long long scaleOff, int rows, int cols,
                     const float* weight, float eps, uint16_t* y, int tiled);
/* y = x - sub (sub may be NULL: y = x) as the tiled fp16 operand of ns2_linear_f16w_tiled
 * ([ceil(rows/64)][cols/64][8][64][8], padding rows zero; cols % 64 == 0): the input of the
 * DiT's patch embedder (the latent tokens) and of its SPRINT projection (the difference of the
 * two residual streams, app/models/nanosaur2.js:236-243, elementwise sub + linear).
 * Additive to the reference interface. */
int ns2_to_tiled_f16(const float* x, int ldx, const float* sub, int ldsub, uint16_t* y, int rows, int cols);
/* ops.glu + gluShader (app/gpu/ops.js:141-148, app/gpu/kernels.js:344-360):
 * y[r, j] = act(x[r, j]) * x[r, I + j] for x [rows, 2I]. */
int ns2_glu(const float* x, float* y, int rows, int I, int act);
/* ns2_glu followed by the ConvRot rotation, written as fp16 (I % 256 == 0), row-major or
 * tiled as in ns2_norm_mod_rotate_f16. */
int ns2_glu_rotate_f16(const float* x, uint16_t* y, int rows, int I, int act, int tiled);
/* ops.elementwise (app/gpu/ops.js:179-185, kernels.js:496-518): op in NS2_EW_*;
 * b is ignored for silu/copy. */
int ns2_elementwise(int op, const float* a, const float* b, float* y, long long n);
/* ops.accumulate (app/gpu/ops.js:188-192): y += a. */
int ns2_accumulate(float* y, const float* a, long long n);
/* The per-block modulation add of the DiT (app/models/nanosaur2.js:190, `elementwise(add,
 * mod, offset)` once per block) batched over blocks: y[r, i] = a[i] + b[r, i] for r < rows,
 * i < n. Additive to the reference interface (one launch instead of one per block). */
int ns2_add_rows(const float* a, const float* b, float* y, int rows, int n);
/* y[c, r] = x[r, c], fp32 [rows, cols] -> [cols, rows]: the latent <-> token layout change
 * around a pass that the reference's forward does on the host (app/models/nanosaur2.js:220-221,
 * 254-255). Additive to the reference interface. */
int ns2_transpose(const float* x, float* y, int rows, int cols);
/* ops.rowSum (app/gpu/ops.js:151-156, kernels.js:362-376): y[n] = scale*sum_r w[r] x[r, n]. */
int ns2_row_sum(const float* x, const float* w, float* y, int rows, int N, float scale);
/* ops.rmsnorm (app/gpu/ops.js:111-117, kernels.js:60-80): y = x * rsqrt(mean x^2 + eps) * w. */
int ns2_rmsnorm(const float* x, const float* w, float* y, int rows, int cols, float eps);
/* The Gemma3 sandwich norms in one launch: x += rmsnorm(a) * w_add (the post-attention /
 * post-MLP norm and the residual add, app/models/gemma3.js:76-77, 87-88 = ops.rmsnorm +
 * ops.accumulate), then, when y is not null, y = rmsnorm(x) * w_out (the next norm: the MLP's
 * pre-norm, the next layer's input norm or the final norm, gemma3.js:80, 62, 92). Rows of
 * `cols` floats; x, a and y must not alias. Additive to the reference interface. */
int ns2_add_rmsnorm(float* x, const float* a, const float* w_add, const float* w_out, float* y, int rows,
                    int cols, float eps);
/* A Gemma3 output projection and the sublayer norms after it, without the [M, N] product in
 * HBM: t = A W^T (+ bias) (ns2_linear_bf16, gemm.js:98-118), then x += rmsnorm(t) * w_add and,
 * when y is not null, y = rmsnorm(x) * w_out (ns2_add_rmsnorm; app/models/gemma3.js:72-80 for
 * the o projection, 83-92 for the down projection). A fp32 [M, lda]; W bf16 [N, K]; x, y fp32
 * [M, N] contiguous, N <= 1024; x must not alias A or y. Additive to the reference interface. */
/* linear (bf16 weight, no LoRA) of a stacked q|k|v projection followed by the per-head norms of
 * two ops.headNorm calls on its rows (Gemma3, app/models/gemma3.js:62-67): C [M, N] = x W^T
 * (+ bias), then heads [0, H1) RMS-normed with w1 and heads [H1, H1 + H2) with w2 (D each), with
 * split-half RoPE on rows < rope_rows when cs is given (ns2_head_norm's table layout); heads past
 * H1 + H2 (the values) as computed. D is 64, 128 or 256; N / D is at most 8 heads. Additive to the
 * reference interface. */
int ns2_linear_bf16_head_norm(const float* A, int lda, const uint16_t* W, const float* bias, float* C, int M, int N,
                              int K, const float* w1, int H1, const float* w2, int H2, int D, const float* cs,
                              long long sin_off, int rope_rows, float eps);
/* ns2_linear_bf16_head_norm with heads [H1, N/D) (the keys and values) stored as fp16 at
 * kv16[m*ldkv + (h - H1)*D + i] (each fp32 result rounded to nearest once) instead of fp32 in
 * C; C receives heads [0, H1) only. kv16 may point into C's rows past column H1*D (ldkv = 2*N):
 * those fp32 columns are not written. Feeds ns2_attention_rows_f16kv. Additive to the reference
 * interface. */
int ns2_linear_bf16_head_norm_f16kv(const float* A, int lda, const uint16_t* W, const float* bias, float* C, int M,
                                    int N, int K, const float* w1, int H1, const float* w2, int H2, int D,
                                    const float* cs, long long sin_off, int rope_rows, float eps, uint16_t* kv16,
                                    int ldkv);
/* A gate/up projection and its GLU without the [M, N] product in HBM: t = A W^T (+ bias), then
 * Y[m][i] = act(t[m][i]) * t[m][N/2 + i] (ns2_linear_bf16 + ns2_glu; the Gemma3 MLP's fused
 * gate/up weight, app/models/gemma3.js:79-82). W bf16 [N, K] with the gate rows first; Y fp32
 * [M, N/2]. Additive to the reference interface. */
int ns2_linear_bf16_glu(const float* A, int lda, const uint16_t* W, const float* bias, float* Y, int M, int N,
                        int K, int act);
/* ns2_linear_bf16_glu followed by the next linear split over the GLU output's 128-column groups
 * (the Gemma3 MLP's down projection, app/models/gemma3.js:79-83), without the [M, N/2] GLU
 * output in HBM: for each group r, with y_r its [M, 128] columns rounded to fp16 (as a linear
 * rounds its input), part[r] [M, Nd] = y_r W_d[:, 128r:128(r+1)]^T, fp32. wd_tiled: W_d [Nd, N/2]
 * as ns2_tile_bf16_weight writes it. The N/256 shares sum to the product without bias;
 * ns2_parts_add_rmsnorm adds them. N % 256 == 0, Nd % 64 == 0. Additive to the reference
 * interface. */
int ns2_linear_bf16_glu_down(const float* A, int lda, const uint16_t* W, const float* bias, int M, int N, int K,
                             int act, const uint16_t* wd_tiled, int Nd, float* part);
/* The Gemma3 layer's linears on the tiled fp16 path (the bf16 weights re-tiled as fp16 by
 * ns2_tile_bf16_weight, the inputs as tiled fp16 operands [ceil(M/64)*64][K] as
 * ns2_parts_add_rmsnorm_tiled or ns2_to_tiled_f16 write them): ns2_linear_bf16_head_norm_f16kv
 * and ns2_linear_bf16_glu_down with the same outputs, up to the fp32 association of the K sums
 * (the inputs and weights rounded to fp16 the same way). K % 64 == 0. Additive to the reference
 * interface. */
int ns2_linear_f16w_tiled_head_norm_f16kv(const uint16_t* At, const uint16_t* Wt, const float* bias, float* C, int M,
                                          int N, int K, const float* w1, int H1, const float* w2, int H2, int D,
                                          const float* cs, long long sin_off, int rope_rows, float eps,
                                          uint16_t* kv16, int ldkv);
int ns2_linear_f16w_tiled_glu_down(const uint16_t* At, const uint16_t* Wt, const float* bias, int M, int N, int K,
                                   int act, const uint16_t* wd_tiled, int Nd, float* part);
int ns2_linear_bf16_add_rmsnorm(const float* A, int lda, const uint16_t* W, const float* bias, float* x,
                                const float* w_add, const float* w_out, float* y, int M, int N, int K,
                                float eps);
/* The same sublayer norms on a product given as `splits` fp32 shares part [splits][M][N] (as
 * ns2_attention_rows_f16kv_oproj writes them): t = sum of the shares in split order (+ bias), then
 * x += rmsnorm(t) * w_add and, when y is not null, y = rmsnorm(x) * w_out (ns2_add_rmsnorm;
 * app/models/gemma3.js:74-79). N <= 1024. Additive to the reference interface. */
int ns2_parts_add_rmsnorm(const float* part, int splits, const float* bias, float* x, const float* w_add,
                          const float* w_out, float* y, int M, int N, float eps);
/* ns2_parts_add_rmsnorm with y written as the tiled fp16 operand of the next linear
 * ([ceil(M/64)*64][N], each value rounded once; rows past M untouched). N % 64 == 0. Additive to
 * the reference interface. */
int ns2_parts_add_rmsnorm_tiled(const float* part, int splits, const float* bias, float* x, const float* w_add,
                                const float* w_out, uint16_t* yt, int M, int N, float eps);

#ifdef __cplusplus
}
#endif

#endif /* NS2_H */
