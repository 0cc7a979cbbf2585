/*
 * anelm_oracle.h -- CPU restatement of the reference's fused layer-op path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: it is used by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg,
 * and by nothing else.  The product (libanelm_hip.so) never links, loads
 * or calls it, and has no CPU fallback.
 *
 * Every function restates one piece of the reference (Lolendorka/ANE-LM)
 * and cites the file:line it follows.  Element counts are size_t/long where
 * the reference uses int; semantics are otherwise unchanged.
 *
 * Pinning (what checks each function against something other than itself)
 * is listed per function below and enforced by tests/test_oracle_*.py.
 */
#ifndef ANELM_ORACLE_H
#define ANELM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar bit conversions: include/ane_lm/common.h:21-75 ----
 * pinned: exhaustive 65,536-pattern tables against an independent exact-real
 * derivation (round-toward-zero to fp16, NaN->Inf) and numpy widening. */
float    orc_bf16_to_f32(uint16_t bf);      /* common.h:21-26 */
uint16_t orc_f32_to_bf16(float f);          /* common.h:28-32 */
float    orc_f16_to_f32(uint16_t h);        /* common.h:35-56 */
uint16_t orc_f32_to_f16(float f);           /* common.h:58-71 (truncating) */
uint16_t orc_bf16_to_f16(uint16_t bf);      /* common.h:73-75 */

/* vector forms: common.h:77-83 (bf16_to_f32_vec, bf16_to_f16_vec), plus the
 * f16 widening the gather needs.  n is size_t (reference: int). */
void orc_bf16_to_f16_vec(uint16_t* out, const uint16_t* in, size_t n, int nthreads);
void orc_bf16_to_f32_vec(float* out, const uint16_t* in, size_t n);
void orc_f16_to_f32_vec(float* out, const uint16_t* in, size_t n);

/* ---- Qwen3.5 norm weights: core/safetensors.cpp:299-306 (load_norm_weight)
 * out = bf16 widened to fp32 (load_bf16_to_f32 :266-281), then out[i] += 1.0f
 * for i < expected_numel, rounded to nearest even.  The reference's loop runs
 * to expected_numel, so a non-positive count widens only.
 * pinned: all 65,536 patterns against an exact-rational round-to-nearest-even
 * of w + 1 (tests/test_oracle_convert.py). */
void orc_norm_weight_vec(float* out, const uint16_t* in, size_t n, long expected_numel);

/* ---- RMSNorm: core/cpu_ops.cpp:25-31 ----
 * ss = sum(x^2); s = 1/sqrtf(ss/dim + eps); out = x*s; out *= w.
 * vDSP_svesq's summation order is unspecified; the oracle uses the
 * correctly rounded sum (double accumulation, rounded once to float).
 * out may alias x.  pinned: constant-row closed form, unit-RMS invariant,
 * fp64 brute force on tiny dims. */
void orc_rmsnorm(float* out, const float* x, const float* w, int dim, float eps);
/* rows x dim, row strides ld_x / ld_out (elements). */
void orc_rmsnorm_rows(float* out, const float* x, const float* w, long rows, int dim,
                      long ld_x, long ld_out, float eps, int nthreads);

/* ---- activations: core/cpu_ops.cpp:7-23, cpu_ops.h:12-13 ----
 * silu: x / (1 + expf(-x));  mul_sigmoid: y / (1 + expf(-z)).
 * pinned: silu(0)=0, silu(-x)=silu(x)-x, silu(ln 3)=0.75 ln 3, large-|x| limits. */
void orc_silu_vec(float* x, size_t n);
void orc_mul_sigmoid(float* y, const float* z, size_t n);
/* SwiGLU in fp32: h = silu(g) * u  (op order core/ane_runtime.cpp:393-395,
 * silu in the cpu_ops.cpp:7-14 divide form, multiply as cpu_ops.cpp:38). */
void orc_silu_mul(float* h, const float* g, const float* u, size_t n, int nthreads);

/* ---- RoPE: models/llm/qwen3.cpp:200-219 (table), :17-52 (apply) ---- */
/* inv_freq[j] = 1.0f / powf(theta, (float)(2j) / (float)rot_dim)  (qwen3.cpp:206-209) */
void orc_rope_inv_freq(float* inv_freq, int rot_dim, float theta);
/* cos/sin[pos*half + j] = cosf/sinf(pos * inv_freq[j])  (qwen3.cpp:210-218)
 * pinned: row 0 is exactly (1,0); inv_freq[0]=1; geometric ratio; matches
 * fp64 trig to 2^-22. */
void orc_rope_table(float* cos_tab, float* sin_tab, int n_pos, int rot_dim, float theta);
/* Qwen3 half-split rotation of nq q-heads and nk k-heads of one token,
 * table row if cos_row/sin_row non-null, else the on-the-fly fallback
 * (qwen3.cpp:28-52).  pinned: pos 0 identity, pair-norm preservation,
 * complex-multiply equivalence, angle additivity. */
void orc_rope_qwen3(float* q, float* k, int nq, int nk, int head_dim, int pos, float theta,
                    const float* cos_row, const float* sin_row);
/* cpu_ops.cpp:56-80 apply_rope_cached: head strides, partial rot_dim; its
 * fallback rotates ADJACENT pairs (cpu_ops.cpp:68-77) unlike its table path. */
void orc_rope_cached(float* q, float* k, int nq, int nk, int head_dim, int q_head_stride,
                     int k_head_stride, int rot_dim, int pos, float theta,
                     const float* cos_row, const float* sin_row);

/* qk-norm then RoPE over T tokens (qwen3.cpp:444-472): q [T, q_ld], k [T, k_ld],
 * per-head rmsnorm with shared gamma wq/wk [head_dim], then the Qwen3 rotation
 * using table row pos[t] when 0 <= pos[t] < tab_len, else the fallback. */
void orc_qknorm_rope(float* q, float* k, long q_ld, long k_ld, const float* wq, const float* wk,
                     const int32_t* pos, const float* cos_tab, const float* sin_tab, int tab_len,
                     float theta, long T, int nq, int nk, int head_dim, float eps, int nthreads);

/* ---- residual add: qwen3.cpp:516, :527 (vDSP_vadd) ---- */
void orc_residual_add(float* x, const float* y, size_t n, int nthreads);

/* ---- embedding gather: qwen3.cpp:498 ----
 * dtype 0 = fp32 table, 1 = fp16 (exact widening common.h:35-56),
 * 2 = bf16 (common.h:21-26).  Returns -1 (nothing written) if any id is
 * outside [0, vocab). */
int orc_embed_gather(float* out, const void* table, int dtype, const int32_t* ids, long n_ids,
                     long hidden, long vocab);

/* ---- softmax: core/cpu_ops.cpp:83-99 ----
 * m = max; x -= m; x = exp(x); s = sum; x *= 1/s.
 * exp is orc_sampler_expf (a <=1 ulp exp with a fixed operation sequence,
 * see below) and the sum is an order-independent 2^-shift fixed-point sum
 * (shift = 63 - ceil(log2 n)) rounded once to float.  Both replace
 * Accelerate's vvexpf / vDSP_sve, whose ulp behaviour and order are
 * unspecified, so that CPU and GPU produce bit-identical probabilities.
 * pinned: uniform logits -> 1/n exactly, 2-element closed form, shift
 * invariance, sum ~ 1, exp accuracy vs fp64. */
float orc_sampler_expf(float x);
void  orc_softmax(float* x, int n);
int   orc_softmax_shift(long n);

/* ---- sample_token: core/sampling.cpp:10-66, sampling.h:7-12 ----
 * logits are not modified (private copy, sampling.cpp:13-14); penalties per
 * unique id in the last ctx entries of recent (ids outside [0,V) skipped);
 * temperature <= 0 -> argmax, first max, r unused; else x *= 1/T, softmax,
 * sequential fp32 CDF walk with cum >= r, V-1 if never reached.
 * probs_out (may be NULL) receives the probabilities when T > 0.
 * pinned: hand-computed known-answer cases (tests/golden/sampler_kat.json). */
int orc_sample_token(const float* logits, int V, float temperature, float rep_penalty, int ctx,
                     float freq_penalty, const int32_t* recent, int n_recent, float r,
                     float* probs_out);
/* the CDF walk alone (sampling.cpp:58-65) on given probabilities */
int orc_cdf_walk(const float* p, int V, float r);

/* ---- KV ring and GQA decode attention ---- */
/* Append one token's k, v rows (kv_stride = n_kv_heads*head_dim floats each)
 * to a ring of `capacity` rows, models/llm/qwen3.cpp:475-488: while
 * len < capacity the slot is start+len (mod capacity) and len grows;
 * afterwards the oldest row (slot start) is overwritten and start advances.
 * Returns the slot written.  pinned: a Python list model of the ring over
 * more appends than the capacity (tests/test_oracle_attention.py). */
int orc_kv_ring_append(float* k_cache, float* v_cache, const float* k, const float* v, int kv_stride,
                       int* start, int* len, int capacity);
/* core/cpu_ops.cpp:173-240 for one token: k_cache / v_cache [capacity,
 * n_kv_heads, head_dim]; the cache_len positions in ring order start,
 * start+1, ... (mod capacity); q head h at q + h*q_head_stride uses kv head
 * h / (n_heads / n_kv_heads); out [n_heads, head_dim].
 *   score_t = fl(dot(q_h, k_t)) * fl(1/sqrtf(head_dim))     :182, :196-209
 *   p = softmax(score)  (orc_softmax, as :211 calls softmax)
 *   out_h = sum_t p_t * v_t, accumulated in ring order     :213-223
 * vDSP_dotpr's summation order is unspecified; the oracle uses the
 * correctly rounded dot (double accumulation).  cache_len <= 0 -> out = 0
 * (:177-180).  pinned: len 1 -> out = v exactly, uniform keys, fp64 brute
 * force with an independent ring enumeration, ring-rotation identity. */
void orc_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                       int n_heads, int n_kv_heads, int head_dim, int q_head_stride, int cache_start,
                       int cache_len, int cache_capacity);

/* ---- Qwen3.5 linear-attention (DeltaNet) ops, core/cpu_ops.cpp:33-39, :100-171 ---- */
/* rmsnorm (eps 1e-6, the default argument) then out = out/(1+expf(-z)),
 * out *= z  (cpu_ops.cpp:33-39).  pinned: z = 0 gives exact zeros,
 * equals rmsnorm * silu(z) in fp64, constant-row closed form. */
void orc_rmsnorm_gated(float* out, const float* x, const float* z, const float* w, int dim);
/* x *= 1/sqrtf(sum x^2 + 1e-12)  (cpu_ops.cpp:105-110; the sum correctly
 * rounded).  pinned: unit norm, exact power-of-two scale invariance,
 * constant-vector closed form, zero vector stays zero. */
void orc_l2_normalize(float* x, int dim);
/* Depthwise causal conv over a ring of the last kernel_size-1 inputs per
 * channel (cpu_ops.cpp:112-150): conv_state [channels, kernel_size-1], the
 * oldest entry at *state_pos; y = sum_j state[(pos+j) mod (K-1)]*w[j] +
 * x*w[K-1], as fused multiply-adds in that order (what clang's default
 * -ffp-contract=on makes of :131 and :140-145 on the reference's arm64
 * target); then the oldest entry becomes x and pos advances.
 * pinned: float64 direct convolution over the input history. */
void orc_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x, const float* w,
                       int channels, int kernel_size);
/* Delta-rule state step (cpu_ops.cpp:152-171): state [key_dim, value_dim];
 * Sk = state^T k; delta = v - Sk; state = decay*state + beta*k*delta^T;
 * y = state^T q.  BLAS summation order is unspecified: the oracle rounds
 * each dot and each updated element once from double.
 * pinned: float64 brute force; decay 1 beta 0 leaves the state; the delta
 * rule recalls v for a unit key. */
void orc_ssm_step(float* y, float* state, const float* q, const float* k, const float* v, float decay,
                  float beta, int key_dim, int value_dim);
/* y = W x, W [out_dim, in_dim] row-major (cpu_ops.cpp:100-103, cblas_sgemv);
 * each dot correctly rounded.  pinned: identity matrix, fp64 brute force. */
void orc_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim);

/* ---- device-resident forward: the ANE contractions and a Qwen3 decode step ---- */
/* fp32 -> fp16 rounded to nearest even (arm64's __fp16 cast at the ANE
 * inputs, core/ane_runtime.cpp:604-612).  pinned: numpy's float16 cast
 * (round to nearest even) over every fp16 boundary and random values. */
uint16_t orc_f32_to_f16_rne(float f);
/* One ANE projection (core/ane_runtime.cpp:265-290 conv as a matvec, with
 * ane_matvec's fp16 input and output, :600-640) for `batch` rows:
 * y16[b,o] = fp16_rne(sum_i x16[b,i] * w16[o,i]) with the sum exact (double
 * accumulation, rounded once).  W [out_dim, in_dim] fp16 bits.
 * pinned: float64 matmul of the same fp16 values. */
void orc_linear_f16(uint16_t* y16, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim,
                    int in_dim);

/* Qwen3 decode step (models/llm/qwen3.cpp:497-564) for `batch` independent
 * sequences, each with its own KV rings (capacity kv_capacity, qwen3.cpp:
 * 227-231), with the reference's ANE projections: weights are the truncating
 * fp16 convert of the bf16 checkpoint (the blobs), activations enter each
 * projection as RNE fp16 and leave it as fp16 (q|k|v fused, o_proj,
 * gate|up, down, LM head); everything else is the oracle functions above
 * (norms, q/k norm + RoPE with the min(max_pos,16384)-row table, ring,
 * attention, SiLU*up in fp32, residual adds).  Per layer the tensors are, in
 * order: q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, gate_proj, up_proj,
 * down_proj, input_layernorm, post_attention_layernorm (bf16 bits). */
typedef struct orc_qwen3_config {
    int hidden, layers, n_q_heads, n_kv_heads, head_dim, intermediate, vocab;
    float rope_theta, rms_eps;
} orc_qwen3_config;
void* orc_qwen3_create(const orc_qwen3_config* c, int batch, int kv_capacity, const uint16_t* embed,
                       const uint16_t* const* layer_tensors, const uint16_t* final_norm,
                       const uint16_t* lm_head);
void orc_qwen3_forward(void* m, const int32_t* ids, const int32_t* pos, float* logits);
void orc_qwen3_free(void* m);

/* ---- one layer of the fused op chain over T tokens, per token as the
 * reference's forward() runs it (qwen3.cpp:502-528):
 *   (1) xn = rmsnorm(x, w_in)                       :503
 *   (2) qk-norm + RoPE on q, k in place             :444-472
 *   (3) x += attn_out; xn = rmsnorm(x, w_post)      :516, :518
 *   (4) h = silu(g) * u                             (fused_ffn, fp32)
 *   (5) x += mlp_out                                :527
 * gammas are fp32 (the configs' fp16 gammas widened exactly). */
void orc_layer_chain(long T, int H, int nq, int nk, int D, int I, float* x, float* xn,
                     const float* attn_out, const float* mlp_out, float* q, float* k,
                     const float* g, const float* u, float* h, const float* w_in,
                     const float* w_post, const float* wq, const float* wk, const int32_t* pos,
                     const float* cos_tab, const float* sin_tab, int tab_len, float theta,
                     float eps, int nthreads);

/* number of OpenMP threads the library would use for nthreads <= 0 */
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
