// Declarations of the names that the integration guide's code uses, so that every
// call it documents can be compiled against the library's real headers
// (include/anelm_hip.h and the ane_lm:: drop-in headers).  Nothing here is
// defined or run: tests/cpp/integration_doc.py wraps each documented block in
// a function of its own and compiles the result with -fsyntax-only, so an
// argument of the wrong type or a wrong argument count fails the build.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>

#include "anelm_hip.h"
#include "ane_lm/convert.h"
#include "ane_lm/cpu_ops.h"
#include "ane_lm/sampling.h"

namespace doc {

constexpr int kLayers = 64;

// the layer loop of a device-resident forward (qwen3.cpp:497-530)
extern float *x, *xn, *xn2, *q, *k, *v, *attn, *mlp, *y, *h, *g, *u, *probs, *logits, *r, *qkv;
extern const void* embed_f16;
extern int32_t *ids, *bad_count, *hist, *hist_len;
extern const int32_t* pos;
extern long T, B, q_ld, k_ld, v_ld, seq_stride, max_batch;
extern int H, V, I, n_layers, nq, nk, layers, cap, qdim, kvdim, qkvdim;
extern const void *w_in[kLayers], *w_post[kLayers], *wq[kLayers], *wk[kLayers], *w_final;
extern float *k_cache[kLayers], *v_cache[kLayers];
extern int32_t *kv_start[kLayers], *kv_len[kLayers];
extern const float *cos_tab, *sin_tab;
extern void* ws;
extern size_t ws_bytes;
extern anelm_sampling_params params;
extern void* s;   // hipStream_t
extern float eps, theta;

// the fused decode step: one layer's device weights, caches and ring-state rows
struct DeviceLayer {
    const uint16_t *Wqkv, *Wo, *Wgu, *Wdown;       // fp16 projections
    uint16_t *Wqkv_t, *Wo_t, *Wgu_t, *Wdown_t;     // the same, tiled (anelm_proj_tile_f16)
    const uint16_t *g_in, *g_post, *g_q, *g_k;     // bf16 gammas
    float *kc, *vc;
    int32_t *start, *len;
};
extern DeviceLayer lw;
extern int32_t *ring_start, *ring_len;   // [layers][max_batch]
extern uint16_t *x16, *attn16, *h16;     // fp16 rows, or tiled past 16 sequences

// the Qwen3.5 linear-attention layer (qwen3_5.cpp:513-549), shown for the
// current layer L
extern int L;
extern float *mixed, *pre_oproj;
extern float* conv_state[kLayers];
extern int32_t* conv_pos[kLayers];
extern int32_t* conv_head_pos[kLayers];   // per (sequence, head)
extern const float* conv_w[kLayers];
extern float* ssm_state[kLayers];
extern const float* norm_w[kLayers];
extern const float *decay, *beta, *z;
extern int ch, nkh, nvh;
extern long qkvz_ld;

// The reference's own variables at the call sites that change one line
// (qwen3.cpp:444-472, :516, :527; safetensors.cpp:335): the parameters of the
// function the documented replacements are compiled in.
struct RefLayerWeights {
    float *q_norm, *k_norm;   // qwen3.cpp:280-285 (fp32)
};
#define ANELM_DOC_CALL_SITE_PARAMS                                                                          \
    float *q_raw, float *k_raw, int nqh, int nkh, int hd, const RefLayerWeights &lw, float eps, int pos,   \
        float theta, const float *rope_cos_row, const float *rope_sin_row, float *x_, const float *y, int H, \
        uint16_t *fp16, const uint16_t *bf16_data, int n

}  // namespace doc
