// Drop-in declarations for the reference's core/cpu_ops.h (Lolendorka/ANE-LM),
// backed by libanelm_hip.so on an MI355X.  Same namespace, names, parameter
// lists and return types as core/cpu_ops.h:10-33; host pointers; each call is
// synchronous and reentrant (thread-local HIP stream and device staging).
// On any device error the call prints the library's message to stderr and
// aborts: there is no CPU fallback.
//
// Every function of core/cpu_ops.h is provided, so core/cpu_ops.cpp can be
// dropped from the build.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace ane_lm {

// core/cpu_ops.h:12-14 (scalar helpers, unchanged: host inline functions)
inline float silu_f(float x) { return x / (1.0f + expf(-x)); }
inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
inline float softplus_f(float x) { return logf(1.0f + expf(x)); }

// core/cpu_ops.h:16-17 -- tmp is accepted and unused
void silu_vec_inplace(float* x, int n, float* tmp);
void mul_sigmoid_inplace(float* y, const float* z, int n, float* tmp);

// core/cpu_ops.h:21 -- out may equal x
void rmsnorm(float* out, const float* x, const float* weight, int dim, float eps = 1e-6f);
// core/cpu_ops.h:22
void rmsnorm_gated(float* out, const float* x, const float* z,
                   const float* weight, int dim);

// core/cpu_ops.h:26-29
void apply_rope_cached(float* q, float* k, int n_q_heads, int n_kv_heads,
                       int head_dim, int q_head_stride, int k_head_stride,
                       int rot_dim, int pos, float theta,
                       const float* cos_row, const float* sin_row);

// core/cpu_ops.h:33
void softmax(float* x, int n);

// core/cpu_ops.h:37
void matvec(float* y, const float* W, const float* x, int out_dim, int in_dim);

// core/cpu_ops.h:41
void l2_normalize(float* x, int dim);

// core/cpu_ops.h:45-46 -- state_pos is the caller's host int, advanced
void conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                   const float* w, int channels, int kernel_size);

// core/cpu_ops.h:49-50
void ssm_step(float* y, float* state, const float* q, const float* k,
              const float* v, float decay, float beta, int key_dim, int value_dim);

// core/cpu_ops.h:53-56 -- caches [cache_capacity, n_kv_heads, head_dim]
// (host memory, staged to the device on every call)
void gqa_attention(float* out, const float* q,
                   const float* k_cache, const float* v_cache,
                   int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                   int cache_start, int cache_len, int cache_capacity);

// Additive entry points for the ops the reference performs inline in
// models/llm/qwen3.cpp (not behind any header there).
namespace hip {
// qwen3.cpp:516 / :527 -- vDSP_vadd(x, y, x)
void residual_add(float* x, const float* y, int n);
// qwen3.cpp:444-472 for one token: per-head rmsnorm of q (nq heads) and k
// (nk heads) with the shared gammas, then the Qwen3 half-split RoPE with
// the table row (cos_row/sin_row, head_dim/2 entries) or, when they are
// null, the on-the-fly fallback at pos.
void qknorm_rope_qwen3(float* q, float* k, int nq, int nk, int head_dim,
                       const float* q_norm, const float* k_norm, float eps,
                       int pos, float theta, const float* cos_row, const float* sin_row);
// SwiGLU h = silu(g) * u in fp32 (the fused_ffn activation,
// core/ane_runtime.cpp:393-395).  h may equal g or u.
void silu_mul(float* h, const float* g, const float* u, int n);
}  // namespace hip

}  // namespace ane_lm
