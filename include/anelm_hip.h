/*
 * anelm_hip.h -- C ABI of the MI355X (gfx950) fused layer-op library
 * (libanelm_hip.so).
 *
 * Replaces the host-side hot path of Lolendorka/ANE-LM: core/cpu_ops
 * (RMSNorm, per-head q/k RMSNorm, RoPE, SiLU/SwiGLU, softmax), the inline
 * ops of models/llm/qwen3.cpp (embedding gather, residual add, the RoPE
 * table), core/sampling (penalties, temperature, softmax, categorical draw)
 * and the bf16->fp16 weight convert of include/ane_lm/common.h.
 *
 * Conventions
 *  - every pointer argument is a DEVICE pointer unless stated otherwise;
 *  - `stream` is a hipStream_t (NULL = the default stream); every call is
 *    asynchronous on it and performs no allocation and no synchronisation;
 *  - element counts and strides are in elements, never bytes;
 *  - return 0 (ANELM_OK) or a negative ANELM_ERR_*; on error nothing was
 *    launched and nothing was written, and anelm_last_error() (per thread)
 *    describes the failure;
 *  - calls are reentrant: no global mutable state besides the per-thread
 *    error string;
 *  - fp32 arithmetic follows the reference's formulas with correctly rounded
 *    division and square root; no fast-math anywhere.
 *
 * The C++ drop-in layer with the reference's own signatures
 * (ane_lm::rmsnorm, ane_lm::sample_token, ...) is declared in
 * ane-lm_amd/host/ane_lm/{cpu_ops,sampling,convert}.h and is built into the
 * same library.
 */
#ifndef ANELM_HIP_H
#define ANELM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANELM_OK             0
#define ANELM_ERR_INVALID  (-1)  /* null pointer, bad size, stride or alignment */
#define ANELM_ERR_RANGE    (-2)  /* a host-visible index out of range */
#define ANELM_ERR_HIP      (-3)  /* the HIP runtime reported an error */
#define ANELM_ERR_WORKSPACE (-4) /* workspace missing or too small */

/* storage types of weights / tables */
#define ANELM_F32  0
#define ANELM_F16  1
#define ANELM_BF16 2
/* further safetensors file dtypes (anelm_st_info) */
#define ANELM_ST_F64 3
#define ANELM_ST_I32 4
#define ANELM_ST_I64 5
#define ANELM_ST_U8  6
#define ANELM_ST_UNKNOWN (-1)

/* Description of the last error on the calling thread ("" if none). */
const char* anelm_last_error(void);
/* Library version, major*10000 + minor*100 + patch. */
int anelm_version(void);

/* ---------------------------------------------------------------- norms */

/* RMSNorm over `rows` rows of `dim` floats:
 *   out[r,:] = (x[r,:] * s) * w,  s = 1/sqrtf(sum(x^2)/dim + eps)
 * Replaces ane_lm::rmsnorm, core/cpu_ops.h:21 / core/cpu_ops.cpp:25-31
 * (callers models/llm/qwen3.cpp:503, :518, :530), batched over rows.
 * w has `dim` entries of type w_dtype (ANELM_F32/F16/BF16).  out may equal x. */
int anelm_rmsnorm(float* out, const float* x, const void* w, int w_dtype, long rows, int dim,
                  long ld_x, long ld_out, float eps, void* stream);

/* The launch geometry that anelm_rmsnorm (16-byte aligned rows) and
 * anelm_layer_ops choose for `rows` rows of `dim` floats: float4 values per
 * lane and lanes per row; 0 float4 per lane names the any-shape kernel (dim
 * not a multiple of 4 or above 16384).  The geometry fixes the order of the
 * sum of squares.  Launches nothing.  No counterpart in the reference. */
int anelm_rmsnorm_geometry(long rows, int dim, int* float4_per_lane, int* threads);

/* anelm_rmsnorm with the result rounded to fp16 (nearest even), the ANE
 * kernels' input conversion (core/ane_runtime.cpp:604-612) fused into the
 * norm: out16 = fp16(rmsnorm(x) * w), the same fp32 values as anelm_rmsnorm
 * (bit-identical to it followed by anelm_f32_to_f16 wherever both take the
 * vector path: dim a multiple of 4, 16-byte aligned rows).  The input of a projection that takes fp16 rows
 * (anelm_proj_f16_x16, anelm_proj_f16_x16_fused); out16 must not overlap x.
 * No counterpart in the reference. */
int anelm_rmsnorm_f16(uint16_t* out16, const float* x, const void* w, int w_dtype, long rows, int dim, long ld_x,
                      long ld_out, float eps, void* stream);
/* anelm_rmsnorm_f16 with out_t in the tiled layout of anelm_proj_tile_f16
 * (rows of x as its rows, dim a multiple of 32): for each 16-row tile and
 * 32-column step, the 16 x 32 block as one contiguous 1 KB piece; rows past
 * `rows` in the last tile are left as they are.  out_t holds
 * anelm_proj_tiled_size(rows, dim) bytes, 16-byte aligned; x 16-byte
 * aligned, ld_x a multiple of 4.  The same fp16 values as anelm_rmsnorm_f16:
 * the input of anelm_proj_f16_tt.  No counterpart in the reference. */
int anelm_rmsnorm_f16_tiled(uint16_t* out_t, const float* x, const void* w, int w_dtype, long rows, int dim,
                            long ld_x, float eps, void* stream);
/* Fused residual add + RMSNorm:  x[r,:] += y[r,:];  out[r,:] = rmsnorm(x[r,:]).
 * Replaces the pair vDSP_vadd(x_, attn_out, x_) + rmsnorm(x_norm_, x_, ...)
 * of models/llm/qwen3.cpp:516-518.  y may equal out (the reference's
 * attn_out aliases x_norm_). */
int anelm_add_rmsnorm(float* x, const float* y, float* out, const void* w, int w_dtype, long rows,
                      int dim, long ld_x, long ld_y, long ld_out, float eps, void* stream);

/* Per-head q/k RMSNorm followed by Qwen3 half-split RoPE, in place, for T
 * tokens.  q[t*q_ld + h*head_dim + d] (h < nq), k likewise with k_ld, nk.
 * wq / wk: head_dim gammas shared by all q (k) heads; NULL skips that norm.
 * pos[t] selects row pos[t] of cos_tab/sin_tab ([tab_len, head_dim/2]) when
 * 0 <= pos[t] < tab_len; otherwise the angle pos*inv_freq[j] is evaluated
 * on the fly with inv_freq[j] = 1/powf(theta, 2j/head_dim) computed on the
 * host exactly as the reference does.
 * Replaces models/llm/qwen3.cpp:444-472 (qk-norm via ane_lm::rmsnorm, then
 * the static apply_rope_qwen3 :28-52, row choice :463-469). */
int anelm_qknorm_rope(float* q, float* k, long q_ld, long k_ld, const void* wq, const void* wk,
                      int w_dtype, const int32_t* pos, const float* cos_tab, const float* sin_tab,
                      int tab_len, float theta, long T, int nq, int nk, int head_dim, float eps,
                      void* stream);

/* The decode step's anelm_qknorm_rope then anelm_kv_ring_append in one
 * launch (models/llm/qwen3.cpp:444-488), head_dim 128: token b of `batch` is
 * sequence b's (position pos[b]); its q heads (q + b*q_ld, nq of them) and k
 * heads (k + b*k_ld, nk) are normalised and rotated in place exactly as
 * anelm_qknorm_rope does, and its k (as rotated) and v (v + b*v_ld, copied)
 * are appended to ring b exactly as anelm_kv_ring_append does.  q, k, v, the
 * caches and the tables 16-byte aligned, strides multiples of 4.  No
 * counterpart in the reference (there the three steps are separate loops). */
int anelm_qknorm_rope_append(float* q, float* k, const float* v, long q_ld, long k_ld, long v_ld, const void* wq,
                             const void* wk, int w_dtype, const int32_t* pos, const float* cos_tab,
                             const float* sin_tab, int tab_len, float theta, long batch, int nq, int nk, float eps,
                             float* k_cache, float* v_cache, int32_t* ring_start, int32_t* ring_len, int capacity,
                             long cache_seq_stride, void* stream);

/* ane_lm::apply_rope_cached semantics (core/cpu_ops.h:26-29,
 * core/cpu_ops.cpp:56-80) for ONE token: heads at q + h*q_head_stride and
 * k + h*k_head_stride, the first rot_dim elements rotated.  With a table row
 * (cos_row/sin_row non-NULL, rot_dim/2 entries) the pairs are (j, j+rot_dim/2);
 * without one the reference's fallback rotates ADJACENT pairs (2i, 2i+1)
 * with freq 1/powf(theta, 2i/rot_dim) and angle pos*freq. */
int anelm_rope_cached(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                      int q_head_stride, int k_head_stride, int rot_dim, int pos, float theta,
                      const float* cos_row, const float* sin_row, void* stream);

/* RoPE table: cos_tab/sin_tab[p*(rot_dim/2) + j] = cos/sin(p * inv_freq[j]),
 * inv_freq as above, for p in [0, n_pos).  Replaces the load-time loop of
 * models/llm/qwen3.cpp:200-219.  rot_dim even, <= 1024. */
int anelm_rope_table(float* cos_tab, float* sin_tab, int n_pos, int rot_dim, float theta,
                     void* stream);

/* The five layer ops of models/llm/qwen3.cpp:502-528 for T tokens in one
 * launch, for a caller that holds all of the layer's op inputs at once (the
 * op chain without contractions between its ops; e.g. decode-shaped chains,
 * whose separate launches are each a few microseconds of latency):
 *   xn_in = rmsnorm(x)*w_in; q, k normalised and rotated in place (head_dim
 *   128, RoPE table required); x += attn; xn_post = rmsnorm(x)*w_post;
 *   h = silu(g)*u; x += mlp.
 * Every output is bit-identical to anelm_rmsnorm, anelm_qknorm_rope,
 * anelm_add_rmsnorm, anelm_silu_mul and anelm_residual_add run in that order
 * on the same buffers (xn_in being the first norm's output, xn_post the
 * second's).  Row-major, contiguous: x, xn_in, xn_post, attn, mlp [T, hidden];
 * q [T, nq*128]; k [T, nk*128]; g, u, h [T, inter]; all 16-byte aligned;
 * gammas of w_dtype (w_in, w_post [hidden]; wq, wk [128]).  hidden and inter
 * multiples of 4, hidden <= 16384.  x is read and written once.  No
 * counterpart in the reference (its ops are separate steps). */
int anelm_layer_ops(float* x, float* xn_in, float* xn_post, const float* attn, const float* mlp, float* q, float* k,
                    float* h, const float* g, const float* u, const void* w_in, const void* w_post, const void* wq,
                    const void* wk, int w_dtype, const int32_t* pos, const float* cos_tab, const float* sin_tab,
                    int tab_len, float theta, long T, int hidden, int nq, int nk, long inter, float eps, void* stream);

/* ---------------------------------------------------------- elementwise */

/* Residual add x[i] += y[i] (one IEEE add; bit-exact).
 * Replaces vDSP_vadd at models/llm/qwen3.cpp:516 and :527. */
int anelm_residual_add(float* x, const float* y, size_t n, void* stream);

/* SwiGLU in fp32: h[r,i] = (g / (1 + expf(-g))) * u  for rows x inter.
 * Op order of the reference's fused_ffn (core/ane_runtime.cpp:393-395) with
 * silu in the core/cpu_ops.cpp:7-14 form.  h may equal g or u. */
int anelm_silu_mul(float* h, const float* g, const float* u, long rows, long inter, long ld_h,
                   long ld_g, long ld_u, void* stream);

/* x[i] = x[i] / (1 + expf(-x[i]))    -- ane_lm::silu_vec_inplace, cpu_ops.h:16 */
int anelm_silu(float* x, size_t n, void* stream);
/* y[i] = y[i] / (1 + expf(-z[i]))    -- ane_lm::mul_sigmoid_inplace, cpu_ops.h:17 */
int anelm_mul_sigmoid(float* y, const float* z, size_t n, void* stream);

/* Embedding gather: out[b,:] = table[ids[b],:] widened exactly to fp32
 * (table_dtype ANELM_F32 copy, ANELM_F16 as f16_to_f32 common.h:35-56 incl.
 * NaN payloads, ANELM_BF16 as bf16_to_f32 common.h:21-26).
 * Replaces the memcpy of models/llm/qwen3.cpp:498, batched.  ids live in
 * device memory, so range errors are reported on the device: a row whose id
 * is outside [0, vocab) is not written and, if bad_count is non-NULL,
 * *bad_count is incremented once for it. */
int anelm_embed_gather(float* out, const void* table, int table_dtype, const int32_t* ids,
                       long n_ids, long hidden, long vocab, int32_t* bad_count, void* stream);

/* ---------------------------------------------------------- conversions */

/* bf16 -> fp16, bit-exact with the reference's TRUNCATING convert
 * (bf16_to_f16_vec, include/ane_lm/common.h:73-83: round toward zero,
 * below 2^-25 -> +-0, overflow and NaN -> +-Inf).  Integer arithmetic only.
 * Replaces the per-weight loop at core/safetensors.cpp:335 (write_ane_blob)
 * and core/ane_runtime.cpp:207 (build_weight_blob).  dst may equal src. */
int anelm_bf16_to_f16(uint16_t* dst, const uint16_t* src, size_t n, void* stream);
/* anelm_bf16_to_f16 over many tensors: tensor i is n[i] elements from src[i]
 * to dst[i] (dst[i] may equal src[i]).  dst, src and n are HOST arrays (of
 * device pointers); up to 128 tensors share one launch, so converting a
 * checkpoint tensor by tensor (core/safetensors.cpp:335 in write_ane_blobs'
 * loop, core/ane_runtime.cpp:207 per weight) costs a few launches, not one
 * per tensor.  Tensors whose pointers are not 16-byte aligned get their own
 * launch.  Bit-identical to anelm_bf16_to_f16 per tensor. */
int anelm_bf16_to_f16_multi(uint16_t* const* dst, const uint16_t* const* src, const size_t* n, int count,
                            void* stream);
/* bf16 -> fp32 (bf16_to_f32_vec, common.h:77-79; used by load_bf16_to_f32,
 * core/safetensors.cpp:266-281). */
int anelm_bf16_to_f32(float* dst, const uint16_t* src, size_t n, void* stream);
/* bf16 -> fp32 plus 1.0f (round to nearest even): the Qwen3.5 (1+w) RMSNorm
 * weight of SafeTensors::load_norm_weight, core/safetensors.cpp:299-306. */
int anelm_bf16_to_f32_plus1(float* dst, const uint16_t* src, size_t n, void* stream);
/* fp16 -> fp32 exact widening (f16_to_f32, common.h:35-56). */
int anelm_f16_to_f32(float* dst, const uint16_t* src, size_t n, void* stream);
/* fp32 -> fp16 rounded to nearest even: the activation conversion at the ANE
 * kernel inputs (core/ane_runtime.cpp:604-612, arm64 __fp16). */
int anelm_f32_to_f16(uint16_t* dst, const float* src, size_t n, void* stream);

/* ---------------------------------------------------- softmax / sampling */

/* Row softmax in place over `rows` rows of n floats at stride ld
 * (ane_lm::softmax, core/cpu_ops.h:33 / core/cpu_ops.cpp:83-99):
 * max, x - max, exp, sum, x * (1/sum).  The exp is a fixed <= 1 ulp
 * sequence of IEEE operations and the sum an exact integer fixed-point sum
 * rounded once, so results do not depend on launch geometry.
 * Needs anelm_softmax_workspace_size(rows, n) bytes of device workspace. */
size_t anelm_softmax_workspace_size(long rows, long n);
int anelm_softmax(float* x, long rows, long n, long ld, void* workspace, size_t workspace_bytes,
                  void* stream);

/* Sampling parameters; field meaning and defaults of ane_lm::SamplingParams
 * (core/sampling.h:7-12): 0.6, 1.2, 256, 0.1. */
typedef struct anelm_sampling_params {
    float temperature;
    float repetition_penalty;
    int   repetition_context_size;
    float frequency_penalty;
} anelm_sampling_params;

/* Batched ane_lm::sample_token (core/sampling.h:14-16, core/sampling.cpp:10-66)
 * over `rows` independent rows of `vocab` logits at stride ld_logits
 * (logits are not modified):
 *  - history row b: hist[b*hist_ld + j], j < (hist_len ? hist_len[b] : hist_ld);
 *    the last repetition_context_size entries are used, ids outside
 *    [0, vocab) ignored; each distinct id gets the repetition penalty once
 *    (l>0 ? l/rep : l*rep, only if rep > 1) then l -= freq*count (if freq > 0);
 *  - temperature <= 0: ids[b] = first argmax, r and probs untouched;
 *  - else x *= 1/T, softmax (as anelm_softmax) written to probs (stride
 *    ld_probs; required, it is also the draw's input), then ids[b] = first i
 *    whose SEQUENTIAL fp32 running sum p[0]+...+p[i] is >= r[b], or vocab-1
 *    if none -- computed exactly, identical to the reference's walk
 *    (sampling.cpp:59-65).
 * r[b] is the uniform draw (the reference's (float)drand48()).
 * Needs anelm_sample_workspace_size(rows, vocab) bytes of device workspace,
 * with any contents (nothing needs clearing).  From 12 sampling rows, with
 * 16-byte aligned logits and probability rows, stages 1-3 run as one launch
 * whose row barriers need the whole grid resident on the GPU at once (the
 * library checks that it fits); a barrier that still waits 0.2 s gives up
 * and that row's id is -1 (not seen in normal operation).  Calls on one
 * workspace are ordered on one stream. */
size_t anelm_sample_workspace_size(long rows, long vocab);
int anelm_sample(int32_t* ids, float* probs, long ld_probs, const float* logits, long ld_logits,
                 long rows, long vocab, const int32_t* hist, long hist_ld,
                 const int32_t* hist_len, const anelm_sampling_params* params, const float* r,
                 void* workspace, size_t workspace_bytes, void* stream);
/* anelm_sample for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the same kernels and results, with the workspace taken from a static
 * 4 MiB device array the library holds on every GPU it runs on until the
 * process ends, so it calls no allocator.  Limit:
 * anelm_sample_workspace_size(rows, vocab) <= 4 MiB (181 rows at a 151936-row
 * vocabulary); larger calls return ANELM_ERR_WORKSPACE.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (on different
 * streams, or from different threads) race and must not be issued.  The
 * first call on a device looks the array's address up (hipGetSymbolAddress).
 * No counterpart in the reference (its sample_token allocates per call). */
int anelm_sample_noalloc(int32_t* ids, float* probs, long ld_probs, const float* logits, long ld_logits,
                         long rows, long vocab, const int32_t* hist, long hist_ld,
                         const int32_t* hist_len, const anelm_sampling_params* params, const float* r,
                         void* stream);

/* ------------------------------------------------ KV ring and attention */

/* Per-sequence KV rings: for sequence b, k_cache/v_cache + b*cache_seq_stride
 * each hold [capacity, n_kv_heads, head_dim] fp32 (the layout of the
 * reference's KVCache, models/llm/qwen3.cpp:227-231); ring_start[b] /
 * ring_len[b] (device int32) name the live rows start, start+1, ...
 * (mod capacity), len of them.  Out-of-range state is clamped on the device
 * (0 <= len <= capacity, start taken mod capacity) so no access leaves the
 * caches. */

/* Appends row b of k and v (n_kv_heads*head_dim floats at k + b*k_ld,
 * v + b*v_ld) to ring b and advances its state, as models/llm/qwen3.cpp:475-488:
 * while len < capacity the row goes to slot start+len (mod capacity) and len
 * grows; afterwards it overwrites slot start and start advances. */
int anelm_kv_ring_append(float* k_cache, float* v_cache, int32_t* ring_start, int32_t* ring_len,
                         const float* k, const float* v, long k_ld, long v_ld, long batch,
                         int n_kv_heads, int head_dim, int capacity, long cache_seq_stride,
                         void* stream);

/* GQA decode attention (ane_lm::gqa_attention, core/cpu_ops.cpp:173-240,
 * core/cpu_ops.h:53-56) for `batch` sequences at once: q head h of sequence b
 * at q + b*q_ld + h*q_head_stride attends over ring b with kv head
 * h / (n_heads/n_kv_heads):
 *   score_t = dot(q_h, k_t) * (1/sqrtf(head_dim)), p = softmax(score),
 *   out[b*out_ld + h*head_dim + d] = sum_t p_t v_t[d];
 * an empty ring gives zeros (cpu_ops.cpp:177-180).  head_dim 64, 128 or 256;
 * n_heads a multiple of n_kv_heads; q and the caches 16-byte aligned with
 * strides that are multiples of 4.  Needs
 * anelm_gqa_workspace_size(batch, n_heads, n_kv_heads, head_dim, capacity)
 * bytes of device workspace (0 is possible: then workspace may be NULL),
 * zero-filled before its first use (e.g. hipMemset once after allocating).
 * That size serves every call with at most `batch` sequences and rings of at
 * most `capacity` rows.  The workspace's last 64th holds per-(sequence, kv
 * head) counters of the chunks of a long ring, at addresses that depend only
 * on workspace_bytes; no call writes partial results there and every call
 * leaves them at zero, so one workspace, passed with the same
 * workspace_bytes, serves calls of any batch, bound or ring length in any
 * order.  Calls that share a workspace must not overlap. */
size_t anelm_gqa_workspace_size(long batch, int n_heads, int n_kv_heads, int head_dim, int capacity);
int anelm_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                        const int32_t* ring_start, const int32_t* ring_len, long batch, int n_heads,
                        int n_kv_heads, int head_dim, long q_ld, int q_head_stride, long out_ld,
                        int capacity, long cache_seq_stride, void* workspace, size_t workspace_bytes,
                        void* stream);
/* anelm_gqa_attention with the outputs rounded to fp16 (nearest even) into
 * out16 (row stride out_ld elements): the o projection's input, rounded once
 * here instead of in every projection workgroup (anelm_proj_f16_x16_fused).
 * Each value equals anelm_gqa_attention's then anelm_f32_to_f16.  No
 * counterpart in the reference. */
int anelm_gqa_attention_f16(uint16_t* out16, const float* q, const float* k_cache, const float* v_cache,
                            const int32_t* ring_start, const int32_t* ring_len, long batch, int n_heads,
                            int n_kv_heads, int head_dim, long q_ld, int q_head_stride, long out_ld, int capacity,
                            long cache_seq_stride, void* workspace, size_t workspace_bytes, void* stream);
/* The ring-state half of anelm_kv_ring_append (models/llm/qwen3.cpp:475-484)
 * for groups x batch rings at once: ring g*group_stride + b (g < groups,
 * b < batch) takes one row, its state advanced as the append does, the
 * caches untouched.  With every layer's rings advanced this way before a
 * decode step, each layer's anelm_gqa_attention_qk makes and stores the new
 * row itself.  No counterpart in the reference. */
int anelm_kv_ring_advance(int32_t* ring_start, int32_t* ring_len, long batch, int groups, long group_stride,
                          int capacity, void* stream);
/* anelm_qknorm_rope_append then anelm_gqa_attention (out_f16 = 0), or
 * anelm_gqa_attention_f16 (out_f16 = 1; with out_f16 = 2 the fp16 outputs in
 * the tiled layout of anelm_proj_tile_f16 with n_heads*128 columns, out
 * 16-byte aligned, out_ld unused: the input of anelm_proj_f16_tt),
 * in one launch, head_dim 128, for rings that anelm_kv_ring_advance has
 * already advanced: the new row's slot is (start + len - 1) mod capacity.
 * q (q + b*q_ld, n_heads heads 128 apart), k and v (k + b*k_ld, v + b*v_ld,
 * n_kv_heads heads) are the raw projection outputs and are not written; the
 * q heads are normalised and rotated on the fly, and k (normalised, rotated)
 * and v are stored into the new slot.  wq and wk are required and the RoPE
 * table must hold at least one row (positions past it use the angle
 * pos*inv_freq[j], as anelm_qknorm_rope does).  Outputs, caches and ring state equal
 * the separate calls' bit for bit (models/llm/qwen3.cpp:444-488 then
 * core/cpu_ops.cpp:173-240).  Workspace as anelm_gqa_attention's with
 * head_dim 128.  No counterpart in the reference. */
int anelm_gqa_attention_qk(void* out, int out_f16, const float* q, const float* k, const float* v, long q_ld,
                           long k_ld, long v_ld, const void* wq, const void* wk, int w_dtype, const int32_t* pos,
                           const float* cos_tab, const float* sin_tab, int tab_len, float theta, float eps,
                           float* k_cache, float* v_cache, const int32_t* ring_start, const int32_t* ring_len,
                           long batch, int n_heads, int n_kv_heads, long out_ld, int capacity,
                           long cache_seq_stride, void* workspace, size_t workspace_bytes, void* stream);
/* anelm_kv_ring_advance of the batch's rings (groups 1), then
 * anelm_gqa_attention_qk, for callers that advance one layer's rings at a
 * time: the ring append and attention of models/llm/qwen3.cpp:475-492 after
 * the q/k norm + RoPE of :444-472, with no precondition on the ring state
 * (anelm_gqa_attention_qk needs rings advanced exactly once since its last
 * call on them).  Arguments as anelm_gqa_attention_qk, ring state writable;
 * every argument and the workspace size are checked before anything is
 * launched, so an error leaves the rings unchanged.  Two launches; outputs,
 * caches and ring state equal the separate calls' bit for bit.  No
 * counterpart in the reference. */
int anelm_gqa_attention_qk_append(void* out, int out_f16, const float* q, const float* k, const float* v,
                                  long q_ld, long k_ld, long v_ld, const void* wq, const void* wk, int w_dtype,
                                  const int32_t* pos, const float* cos_tab, const float* sin_tab, int tab_len,
                                  float theta, float eps, float* k_cache, float* v_cache, int32_t* ring_start,
                                  int32_t* ring_len, long batch, int n_heads, int n_kv_heads, long out_ld,
                                  int capacity, long cache_seq_stride, void* workspace, size_t workspace_bytes,
                                  void* stream);
/* anelm_gqa_attention for callers that know an upper bound on every ring's
 * length (len_bound >= ring_len[b] for all b; e.g. the tokens decoded since
 * the rings were emptied): only ceil(len_bound / chunk) chunks per sequence
 * are launched (at least 64 positions each), and with one chunk the
 * workgroup writes the output itself, with no partials to merge.  A ring
 * longer than len_bound is attended over its first positions only: those of
 * the launched chunks, whose last to finish merges them.  No counterpart in
 * the reference (its loop already runs over the live rows only,
 * core/cpu_ops.cpp:186-188). */
int anelm_gqa_attention_bounded(float* out, const float* q, const float* k_cache, const float* v_cache,
                                const int32_t* ring_start, const int32_t* ring_len, long batch, int n_heads,
                                int n_kv_heads, int head_dim, long q_ld, int q_head_stride, long out_ld,
                                int capacity, long cache_seq_stride, int len_bound, void* workspace,
                                size_t workspace_bytes, void* stream);
/* The reference's own single-sequence form, with the ring state as host
 * integers (its exact argument list, core/cpu_ops.h:53-56); caches
 * [cache_capacity, n_kv_heads, head_dim]; out [n_heads, head_dim].
 * cache_len <= 0 gives zeros; cache_len > cache_capacity or a start outside
 * [0, capacity) is ANELM_ERR_RANGE.  Workspace as anelm_gqa_attention with
 * batch 1. */
int anelm_gqa_attention_ring(float* out, const float* q, const float* k_cache, const float* v_cache,
                             int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                             int cache_start, int cache_len, int cache_capacity, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ------------------------------ Qwen3.5 linear-attention ops and matvec */

/* Gated RMSNorm of rows x heads vectors of `dim` (vector (r, h) at
 * r*ld + h*dim of each operand): out = rmsnorm(x)*w (the anelm_rmsnorm
 * rounding steps), then out = out/(1 + expf(-z)), then out *= z.  Replaces ane_lm::rmsnorm_gated (core/cpu_ops.cpp:33-39,
 * cpu_ops.h:22; the reference passes no eps, so its default 1e-6 applies),
 * called per value head at models/llm/qwen3_5.cpp:545-549.  out may equal x. */
int anelm_rmsnorm_gated(float* out, const float* x, const float* z, const void* w, int w_dtype, long rows,
                        int heads, int dim, long ld_x, long ld_z, long ld_out, float eps, void* stream);

/* v = (v * (1/sqrtf(sum v^2 + 1e-12))) * scale, in place, for the rows x
 * heads vectors v of `dim` at x + r*ld + h*dim (ane_lm::l2_normalize,
 * core/cpu_ops.cpp:105-110, cpu_ops.h:41).  scale = 1
 * is the reference function itself (the second product is exact); the
 * q path of models/llm/qwen3_5.cpp:528-531 passes 1/sqrtf(key_dim). */
int anelm_l2_normalize(float* x, long rows, int heads, int dim, long ld, float scale, void* stream);

/* Causal depthwise conv1d step for `batch` sequences (ane_lm::conv1d_update,
 * core/cpu_ops.cpp:112-150, cpu_ops.h:45-46): per sequence b a ring
 * conv_state + b*state_stride of [channels, kernel_size-1] past inputs whose
 * oldest entry is at state_pos[b] (device int32); y = sum_j
 * state[(pos+j) mod (K-1)]*w[c*K+j] + x*w[c*K+K-1] as fused multiply-adds
 * in that order, then the oldest entry becomes x and state_pos[b] advances.
 * A state_pos outside [0, K-1) is taken as 0. */
int anelm_conv1d_update(float* y, float* conv_state, int32_t* state_pos, const float* x, const float* w,
                        long batch, int channels, int kernel_size, long ld_x, long ld_y, long state_stride,
                        void* stream);

/* The decode step's conv1d update, SiLU and q/k L2 normalisation in one
 * launch (models/llm/qwen3_5.cpp:513-531; kernel size 4, 128-wide key heads):
 * anelm_conv1d_update, then anelm_silu over all channels, then
 * anelm_l2_normalize of the n_key_heads q heads (channels [0, 128*nkh), times
 * q_scale) and of the k heads (the next 128*nkh channels, scale 1).  Each
 * output is bit-identical to the three calls'.  channels a multiple of 128;
 * w 16-byte aligned.  No counterpart in the reference, which runs the steps
 * one after the other. */
int anelm_conv1d_silu_l2norm(float* y, float* conv_state, int32_t* state_pos, const float* x, const float* w,
                             long batch, int channels, int n_key_heads, long ld_x, long ld_y, long state_stride,
                             float q_scale, void* stream);

/* Delta-rule state step (ane_lm::ssm_step, core/cpu_ops.cpp:152-171,
 * cpu_ops.h:49-50) for `batch` sequences x n_heads value heads: head h of
 * sequence b has state + b*state_stride + h*key_dim*value_dim
 * ([key_dim, value_dim] row-major), q/k from key head h/(n_heads/n_key_heads)
 * at q/k + b*ld_qk, v at v + b*ld_v + h*value_dim, decay/beta[b*n_heads+h]:
 *   Sk = S^T k; delta = v - Sk; S = decay*S + beta*k*delta^T; y = S^T q.
 * The loop of models/llm/qwen3_5.cpp:524-543 in one launch.  key_dim 64, 128
 * or 256; value_dim 64 or 128; state 16-byte aligned. */
int anelm_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                   const float* decay, const float* beta, long batch, int n_heads, int n_key_heads,
                   int key_dim, int value_dim, long ld_qk, long ld_v, long ld_y, long state_stride,
                   void* stream);
/* anelm_ssm_step with anelm_rmsnorm_gated applied to each head's y
 * (models/llm/qwen3_5.cpp:545-549, gate z at z + b*ld_z + h*value_dim, weight
 * norm_w [value_dim] of w_dtype) before it is stored: out = rmsnorm(y)*w,
 * then out/(1 + expf(-z)), then out*z, bit-identical to the two calls; y
 * itself is not stored.  No counterpart in the reference. */
int anelm_ssm_step_gated_norm(float* out, float* state, const float* q, const float* k, const float* v,
                              const float* decay, const float* beta, const float* z, const void* norm_w, int w_dtype,
                              long batch, int n_heads, int n_key_heads, int key_dim, int value_dim, long ld_qk,
                              long ld_v, long ld_z, long ld_out, long state_stride, float eps, void* stream);

/* The decode step's whole linear-attention core (models/llm/qwen3_5.cpp:513-549)
 * in one launch, for n_heads key heads = n_heads value heads of 128:
 * anelm_conv1d_silu_l2norm on x ([q heads | k heads | v], 3*128*n_heads
 * channels; conv_w [channels, 4], 16-byte aligned; conv_state per sequence
 * [channels, 3] at conv_state + b*conv_state_stride), then
 * anelm_ssm_step_gated_norm on its q, k, v.  out and the state are
 * bit-identical to those two calls'; the conv's q, k, v are not stored.  The
 * ring position is kept per (sequence, head): head_pos [batch*n_heads], each
 * advanced by one (heads of a sequence stay equal when they start equal; an
 * out-of-range value is taken as 0).  No counterpart in the reference. */
int anelm_conv_ssm_step_gated_norm(float* out, float* state, float* conv_state, int32_t* head_pos,
                                   const float* x, const float* conv_w, const float* decay, const float* beta,
                                   const float* z, const void* norm_w, int w_dtype, long batch, int n_heads, long ld_x,
                                   long ld_z, long ld_out, long state_stride, long conv_state_stride, float q_scale,
                                   float eps, void* stream);

/* y = W x, W [out_dim, in_dim] row-major fp32 (ane_lm::matvec,
 * core/cpu_ops.cpp:100-103, cpu_ops.h:37; the reference's CPU LM head and
 * DeltaNet a/b projections, models/llm/qwen3_5.cpp:509-510, :689). */
int anelm_matvec(float* y, const float* W, const float* x, long out_dim, int in_dim, void* stream);

/* ------------------------------------------- safetensors and ANE weight blobs */

/* A safetensors file opened for reading (core/safetensors.h:27-59,
 * core/safetensors.cpp:193-244): the file is memory-mapped and its JSON
 * header parsed (every tensor, no count limit; "__metadata__" skipped;
 * names are the raw text between the key's quotes, as the reference keeps
 * them).  A tensor whose data_offsets disagree with dtype x shape or leave
 * the file is an error.  NULL on error (anelm_last_error). A handle is not
 * thread-safe; host calls, they may allocate. */
typedef struct anelm_st anelm_st;
anelm_st* anelm_st_open(const char* path);
void anelm_st_close(anelm_st* st);
long anelm_st_count(const anelm_st* st);
/* index of the tensor with this name, or -1 (SafeTensors::find, :246-253) */
long anelm_st_find(const anelm_st* st, const char* name);
/* name (valid until close), dtype (ANELM_F32/F16/BF16/ST_*), ndims, shape
 * (up to 8 entries), byte offset in the data block and byte size; any output
 * pointer may be NULL. */
int anelm_st_info(const anelm_st* st, long i, const char** name, int* dtype, int* ndims, int64_t* shape,
                  uint64_t* offset, uint64_t* nbytes);
/* host pointer to tensor i's bytes in the mapping (SafeTensors::data / get_bf16_ptr) */
const void* anelm_st_host_data(const anelm_st* st, long i);
/* Tensor i into DEVICE memory dst as dst_dtype: its own dtype (a copy; the
 * reference's load_f32_direct :283-297), or for a BF16 tensor ANELM_F32
 * (exact widening on the device: load_bf16_to_f32 :266-281) or ANELM_F16
 * (the truncating convert on the device, the blobs' data).  Staged through
 * pinned memory on `stream`; returns when the tensor is in place. */
int anelm_st_load(const anelm_st* st, long i, void* dst, int dst_dtype, void* stream);
/* The Qwen3.5 (1+w) norm weight into DEVICE memory dst as fp32
 * (SafeTensors::load_norm_weight, core/safetensors.cpp:299-306): BF16 tensor i
 * widened and offset by 1.0f on the device.  expected_numel > 0 must equal the
 * tensor's element count (else ANELM_ERR_INVALID, the reference's "Shape
 * mismatch" null return); as in the reference, whose offset loop runs to
 * expected_numel, a non-positive count loads the widened weight without the
 * offset.  A tensor that is not BF16 is an error (the reference would read
 * its bytes as bf16). */
int anelm_st_load_norm(const anelm_st* st, long i, float* dst, long expected_numel, void* stream);

/* The 128-byte ANE blob header for num_elements fp16 values
 * (core/safetensors.cpp:322-331, core/ane_runtime.cpp:199-205). */
void anelm_ane_blob_header(uint8_t* header128, uint64_t num_elements);
/* The `convert` command (SafeTensors::write_ane_blobs, core/safetensors.cpp:
 * 345-383): every BF16 tensor becomes <output_dir>/<name, '.' -> '/'>.bin =
 * header + truncating fp16 data (converted on the GPU), directories created
 * as needed.  Returns the number of blobs written or a negative status. */
long anelm_write_ane_blobs(const char* safetensors_path, const char* output_dir, void* stream);

/* ------------------------------ contractions and the device-resident step */

/* One ANE projection for `batch` rows (the conv-as-matvec kernels of
 * core/ane_runtime.cpp:265-408 with ane_matvec's fp16 interface, :600-640):
 * y16[b, o] = fp16(sum_i x16[b, i] * W16[o, i]), W16 [out_dim, in_dim]
 * row-major fp16, fp32 accumulation, one rounding to nearest.  Any shape
 * and alignment; in_dim a multiple of 32 with 16-byte aligned rows takes the
 * MFMA kernels (past 16 rows against a long W, x staged in LDS so each weight
 * row is read once for every row of x). */
int anelm_linear_f16(uint16_t* y16, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim, int in_dim,
                     long ld_x, long ld_y, void* stream);

/* The same projection with the conversions fused (decode batches):
 * y[b, o] = fp16(sum_i fp16_rne(x[b, i]) * W16[o, i]) stored as fp32, x fp32;
 * each weight is read once on the fast paths: in_dim a multiple of 32 (any
 * batch), or batch <= 8 and in_dim a multiple of 8, with ld_x a multiple of
 * 4 and x, W16 16-byte aligned.  Other shapes take a slow any-shape kernel.
 * y must not overlap x. */
int anelm_proj_f16(float* y, const float* x, const uint16_t* w16, long batch, int out_dim, int in_dim, long ld_x,
                   long ld_y, void* stream);
/* anelm_proj_f16 with x already rounded to fp16 (x16 [batch, in_dim], row
 * stride ld_x a multiple of 8, e.g. from anelm_f32_to_f16): for larger
 * batches, where rounding x once beats rounding it in every workgroup.
 * in_dim a multiple of 32; y must not overlap x16.  No counterpart in the
 * reference (the ANE runtime has no batched projection). */
int anelm_proj_f16_x16(float* y, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim, int in_dim,
                       long ld_x, long ld_y, void* stream);

/* Decode-step projections (fp32 x, in_dim a multiple of 32) with the
 * neighbouring layer ops of models/llm/qwen3.cpp:497-530 fused in, so a
 * layer is 7 launches instead of 13.  Any batch; past 16 rows
 * anelm_rmsnorm_f16 with anelm_proj_f16_x16_fused is faster where a norm
 * precedes the projection.  With p the rounded projection of
 * anelm_proj_f16:
 *   norm_bf16 != NULL: x is first replaced by rmsnorm(x) * norm_bf16
 *     (core/cpu_ops.cpp:25-31 with eps; norm_bf16 [in_dim], 16-byte aligned);
 *   ANELM_PROJ_STORE:  y = p;
 *   ANELM_PROJ_ADD:    y = y + p (the residual add);
 *   ANELM_PROJ_SWIGLU: W16 holds out_dim gate rows then out_dim up rows, and
 *     y = silu(p_gate) * p_up (the SwiGLU of core/ane_runtime.cpp:393-395 in
 *     the fp32 form of core/cpu_ops.cpp:7-14);
 *   ANELM_PROJ_SWIGLU_F16: the same rounded to fp16 (nearest even) and
 *     stored as fp16 bits: the down projection's input (anelm_proj_f16_x16_fused).
 * y is fp32, or fp16 with ANELM_PROJ_SWIGLU_F16; ld_y counts its elements.
 * y must not overlap x.  Each result equals the separate kernels' to within
 * the RMSNorm's summation order.  No counterpart in the reference: the ANE runtime fuses
 * these inside its own fp16 programs. */
#define ANELM_PROJ_STORE 0
#define ANELM_PROJ_ADD 1
#define ANELM_PROJ_SWIGLU 2
#define ANELM_PROJ_SWIGLU_F16 3
int anelm_proj_f16_fused(void* y, const float* x, const uint16_t* w16, long batch, int out_dim, int in_dim,
                         long ld_x, long ld_y, const uint16_t* norm_bf16, float eps, int epilogue, void* stream);
/* The epilogues of anelm_proj_f16_fused on inputs already rounded to fp16
 * (x16 [batch, in_dim], row stride ld_x a multiple of 8: anelm_rmsnorm_f16's
 * output, the attention's fp16 output, or a previous ANELM_PROJ_SWIGLU_F16),
 * any batch: half the activation bytes of fp32 rows, and no rounding in
 * every workgroup.  y is fp32 (STORE, ADD, SWIGLU) or, with
 * ANELM_PROJ_SWIGLU_F16, fp16: the SwiGLU result rounded to nearest even,
 * i.e. the down projection's input; ld_y counts y's elements; y must not
 * overlap x16.  in_dim a multiple of 32.  No counterpart in the reference
 * (see anelm_proj_f16_fused). */
int anelm_proj_f16_x16_fused(void* y, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim,
                             int in_dim, long ld_x, long ld_y, int epilogue, void* stream);

/* An fp16 W in a tiled layout for streaming it against many rows of x:
 * for each 16-row tile and 32-input step, the 16 x 32 block as one
 * contiguous 1 KB piece in the MFMA operand order, rows past out_dim zero,
 * so that every 16-byte-per-lane weight load reads 1 KB in a row instead of
 * 64 bytes from each of 16 rows a row pitch apart.  anelm_proj_tiled_size
 * gives its bytes (0 unless in_dim is a multiple of 32); anelm_proj_tile_f16
 * writes it from the row-major W16 [out_dim, in_dim] (16-byte aligned, not
 * overlapping; asynchronous).  anelm_proj_f16_x16_tiled is
 * anelm_proj_f16_x16_fused on the tiled copy, every epilogue, plus
 * ANELM_PROJ_STORE_F16 (the projection rounded to fp16, the ANE's own
 * output); past 16 rows it runs the same kernels on the same operands, so
 * its outputs are bit-identical to anelm_proj_f16_x16_fused's on the
 * row-major W.  in_dim a multiple of 32, ld_x a multiple of 8; for the
 * SwiGLU the tiled W holds the 2*out_dim rows (gate, then up) and out_dim is
 * a multiple of 16.  No counterpart in the reference: the ANE runtime splits
 * its weights into blobs of its own format (core/ane_runtime.cpp:265-408);
 * this is the same contraction laid out for coalesced HBM streaming. */
#define ANELM_PROJ_STORE_F16 4
size_t anelm_proj_tiled_size(int out_dim, int in_dim);
int anelm_proj_tile_f16(uint16_t* w_tiled, const uint16_t* w16, int out_dim, int in_dim, void* stream);
int anelm_proj_f16_x16_tiled(void* y, const uint16_t* x16, const uint16_t* w_tiled, long batch, int out_dim,
                             int in_dim, long ld_x, long ld_y, int epilogue, void* stream);
/* anelm_proj_f16_x16_tiled with x in the tiled layout too (x_t: batch rows,
 * in_dim columns, from anelm_rmsnorm_f16_tiled, anelm_gqa_attention_qk with
 * out_f16 = 2 or a previous ANELM_PROJ_SWIGLU_F16_TILED), so that every
 * activation load also reads 1 KB in a row.  Every epilogue of
 * anelm_proj_f16_x16_tiled, plus ANELM_PROJ_SWIGLU_F16_TILED: the fp16
 * SwiGLU result written in the tiled layout (batch rows, out_dim columns, a
 * multiple of 32; ld_y unused), the input of the next anelm_proj_f16_tt.
 * The MFMA kernels of anelm_proj_f16_x16_fused on the same operands: outputs
 * bit-identical to it past 16 rows.  x_t and W 16-byte aligned, in_dim a
 * multiple of 32.  No counterpart in the reference. */
#define ANELM_PROJ_SWIGLU_F16_TILED 5
int anelm_proj_f16_tt(void* y, const uint16_t* x_t, const uint16_t* w_t, long batch, int out_dim, int in_dim,
                      long ld_y, int epilogue, void* stream);

/* Qwen3 model shape (the config.json fields of models/llm/qwen3.cpp:55-80);
 * head_dim must be 128 (every Qwen3 size). */
typedef struct anelm_qwen3_config {
    int hidden, layers, n_q_heads, n_kv_heads, head_dim, intermediate, vocab;
    float rope_theta, rms_eps;
} anelm_qwen3_config;
/* A Qwen3 checkpoint loaded into HBM for device-resident decoding
 * (models/llm/qwen3.cpp:150-300): projections as the truncating fp16 convert
 * (the reference's ANE blobs), the embedding and norms as bf16 (widened
 * exactly on use), the LM head from lm_head.weight or, when absent, the tied
 * embedding; per layer a KV ring of kv_capacity rows for each of max_batch
 * sequences.  Host object; loading allocates and synchronises `stream`. */
typedef struct anelm_qwen3 anelm_qwen3;
anelm_qwen3* anelm_qwen3_load(const char* safetensors_path, const anelm_qwen3_config* cfg, int max_batch,
                              int kv_capacity, void* stream);
void anelm_qwen3_free(anelm_qwen3* model);
/* Empties every KV ring (not for graph capture: it records memsets). */
int anelm_qwen3_reset(anelm_qwen3* model, void* stream);
/* One decode step (Qwen3Model::forward, models/llm/qwen3.cpp:497-564) for
 * `batch` sequences: token ids[b] at position pos[b] (device int32) appended
 * to sequence b's rings; logits [batch, ld_logits] fp32 (device) receive the
 * LM head's fp16 outputs widened.  Asynchronous on `stream`; bad ids are
 * counted in *bad_ids (device, may be NULL) and leave their rows unset. */
int anelm_qwen3_forward(anelm_qwen3* model, const int32_t* ids, const int32_t* pos, long batch, float* logits,
                        long ld_logits, int32_t* bad_ids, void* stream);

#ifdef __cplusplus
}
#endif
#endif
