// Device-resident Qwen3 decode step: the forward glue of
// models/llm/qwen3.cpp:497-564 with every activation kept in HBM, the
// library's layer-op kernels between the contractions, and the ANE
// contractions (core/ane_runtime.cpp:265-408: fused q|k|v, o_proj,
// gate|up -> down, the LM head) as fp16 projections with fp32 accumulation,
// all hand-written (projection.hip: dot kernels for a few rows, MFMA tiles
// beyond, and an any-shape kernel; no vendor BLAS).  The
// ANE's interface numerics are kept: weights are the truncating fp16 convert
// of the bf16 checkpoint (the blobs), activations enter a projection as
// round-to-nearest fp16 and leave it as fp16 (core/ane_runtime.cpp:600-640).
// The RMSNorms, residual adds and the SwiGLU are fused into the
// projections: up to 16 sequences as the projections' own prologue and
// epilogues (5 library calls per layer instead of 12), past that with the
// norms writing the projections' fp16 inputs (7 calls).  The q/k norm, RoPE,
// ring append and attention are one kernel throughout, after one launch at
// the start of the step has advanced every layer's rings.
//
// A step processes one token of each of `batch` sequences; every sequence
// has its own KV ring per layer (qwen3.cpp:227-231, 475-488).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "anelm_common.hpp"

using anelm::fail;
using anelm::clear_error;


namespace {

constexpr int kRopeRows = 16384;   // min(max_position_embeddings, 16384), qwen3.cpp:201

struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);   // teardown: nothing left to report to
    }
};

}  // namespace

struct anelm_qwen3 {
    anelm_qwen3_config c{};
    int max_batch = 0, cap = 0, qdim = 0, kvdim = 0, qkvdim = 0;
    std::vector<DevBuf*> bufs;   // every device allocation, freed at the end
    // weights
    uint16_t* embed = nullptr;       // bf16 [V, H] (widened exactly by the gather)
    uint16_t* final_norm = nullptr;  // bf16 [H]
    uint16_t* lm16 = nullptr;        // fp16 [V, H]
    uint16_t* lm_tiled = nullptr;    // the same in anelm_proj_tile_f16's layout, past 16 sequences (or null)
    struct Layer {
        uint16_t *qkv16, *o16, *gu16, *down16;   // fp16 projections
        // the same in anelm_proj_tile_f16's layout, past 16 sequences (or null)
        uint16_t *qkv_t = nullptr, *o_t = nullptr, *gu_t = nullptr, *down_t = nullptr;
        uint16_t *qn, *kn, *w_in, *w_post;       // bf16 gammas
        float *kc, *vc;                          // [max_batch][cap][kvdim]
        int32_t *start, *len;                    // [max_batch], rows of ring_start / ring_len
    };
    std::vector<Layer> layers;
    int32_t *ring_start = nullptr, *ring_len = nullptr;   // [layers][max_batch]
    float *cos_tab = nullptr, *sin_tab = nullptr;
    // activations
    float *x, *xn, *qkv, *attn, *o, *gu, *h;
    uint16_t *a16, *y16;
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;


    void* alloc(size_t bytes) {
        DevBuf* d = new DevBuf();
        if (hipMalloc(&d->p, bytes ? bytes : 16) != hipSuccess) {
            delete d;
            return nullptr;
        }
        bufs.push_back(d);
        return d->p;
    }
    ~anelm_qwen3() {
        for (DevBuf* d : bufs) delete d;
    }
};

namespace {

// tensor `name` of the checkpoint into device memory as dtype, with a shape check
int load_tensor(anelm_st* st, const char* name, const std::vector<int64_t>& shape, void* dst, int dtype,
                void* stream) {
    const long i = anelm_st_find(st, name);
    if (i < 0) return fail(ANELM_ERR_INVALID, "qwen3_load: tensor %s not found", name);
    int dt, nd;
    int64_t sh[8];
    anelm_st_info(st, i, nullptr, &dt, &nd, sh, nullptr, nullptr);
    if (dt != ANELM_BF16) return fail(ANELM_ERR_INVALID, "qwen3_load: %s is not BF16", name);
    bool ok = nd == (int)shape.size();
    for (int d = 0; ok && d < nd; d++) ok = sh[d] == shape[d];
    if (!ok) return fail(ANELM_ERR_INVALID, "qwen3_load: %s has an unexpected shape", name);
    return anelm_st_load(st, i, dst, dtype, stream);
}

}  // namespace

extern "C" anelm_qwen3* anelm_qwen3_load(const char* path, const anelm_qwen3_config* cfg, int max_batch,
                                         int kv_capacity, void* stream) {
    clear_error();
    if (!path || !cfg || max_batch <= 0 || kv_capacity <= 0) {
        fail(ANELM_ERR_INVALID, "qwen3_load: bad arguments");
        return nullptr;
    }
    const anelm_qwen3_config& c = *cfg;
    if (c.hidden <= 0 || c.layers <= 0 || c.n_q_heads <= 0 || c.n_kv_heads <= 0 || c.intermediate <= 0 ||
        c.vocab <= 0 || c.head_dim != 128 ||   // every Qwen3 size; the fused q/k + attention kernel's width
        c.n_q_heads % c.n_kv_heads || c.hidden % 4 || c.intermediate % 4) {
        fail(ANELM_ERR_INVALID, "qwen3_load: unsupported configuration");
        return nullptr;
    }
    anelm_st* st = anelm_st_open(path);
    if (!st) return nullptr;
    anelm_qwen3* m = new anelm_qwen3();
    m->c = c;
    m->max_batch = max_batch;
    m->cap = kv_capacity;
    const long H = c.hidden, D = c.head_dim, I = c.intermediate, V = c.vocab, B = max_batch;
    m->qdim = c.n_q_heads * c.head_dim;
    m->kvdim = c.n_kv_heads * c.head_dim;
    m->qkvdim = m->qdim + 2 * m->kvdim;
    int rc = ANELM_OK;
    auto bail = [&](const char* what) {
        if (rc == ANELM_OK) rc = fail(ANELM_ERR_HIP, "qwen3_load: %s", what);
        anelm_st_close(st);
        delete m;
        return (anelm_qwen3*)nullptr;
    };
#define ALLOC(ptr, T, n)                                                   \
    do {                                                                   \
        ptr = static_cast<T*>(m->alloc((size_t)(n) * sizeof(T)));          \
        if (!ptr) return bail("out of device memory");                     \
    } while (0)
    ALLOC(m->embed, uint16_t, V * H);
    ALLOC(m->final_norm, uint16_t, H);
    ALLOC(m->lm16, uint16_t, V * H);
    if ((rc = load_tensor(st, "model.embed_tokens.weight", {V, H}, m->embed, ANELM_BF16, stream)) ||
        (rc = load_tensor(st, "model.norm.weight", {H}, m->final_norm, ANELM_BF16, stream)))
        return bail("");
    const bool tied = anelm_st_find(st, "lm_head.weight") < 0;   // qwen3.cpp:259-263, :383
    if ((rc = load_tensor(st, tied ? "model.embed_tokens.weight" : "lm_head.weight", {V, H}, m->lm16, ANELM_F16,
                          stream)))
        return bail("");
    m->layers.resize(c.layers);
    ALLOC(m->ring_start, int32_t, (long)c.layers * B);
    ALLOC(m->ring_len, int32_t, (long)c.layers * B);
    char name[256];
    for (int L = 0; L < c.layers; L++) {
        anelm_qwen3::Layer& l = m->layers[L];
        ALLOC(l.qkv16, uint16_t, (long)m->qkvdim * H);
        ALLOC(l.o16, uint16_t, H * m->qdim);
        ALLOC(l.gu16, uint16_t, 2 * I * H);
        ALLOC(l.down16, uint16_t, H * I);
        ALLOC(l.qn, uint16_t, D);
        ALLOC(l.kn, uint16_t, D);
        ALLOC(l.w_in, uint16_t, H);
        ALLOC(l.w_post, uint16_t, H);
        ALLOC(l.kc, float, B * m->cap * m->kvdim);
        ALLOC(l.vc, float, B * m->cap * m->kvdim);
        l.start = m->ring_start + (long)L * B;
        l.len = m->ring_len + (long)L * B;
        struct Item {
            const char* n;
            std::vector<int64_t> shape;
            void* dst;
            int dt;
        } items[] = {
            {"self_attn.q_proj.weight", {m->qdim, H}, l.qkv16, ANELM_F16},
            {"self_attn.k_proj.weight", {m->kvdim, H}, l.qkv16 + (long)m->qdim * H, ANELM_F16},
            {"self_attn.v_proj.weight", {m->kvdim, H}, l.qkv16 + (long)(m->qdim + m->kvdim) * H, ANELM_F16},
            {"self_attn.o_proj.weight", {H, m->qdim}, l.o16, ANELM_F16},
            {"self_attn.q_norm.weight", {D}, l.qn, ANELM_BF16},
            {"self_attn.k_norm.weight", {D}, l.kn, ANELM_BF16},
            {"mlp.gate_proj.weight", {I, H}, l.gu16, ANELM_F16},
            {"mlp.up_proj.weight", {I, H}, l.gu16 + I * H, ANELM_F16},
            {"mlp.down_proj.weight", {H, I}, l.down16, ANELM_F16},
            {"input_layernorm.weight", {H}, l.w_in, ANELM_BF16},
            {"post_attention_layernorm.weight", {H}, l.w_post, ANELM_BF16},
        };
        for (const Item& it : items) {
            snprintf(name, sizeof(name), "model.layers.%d.%s", L, it.n);
            if ((rc = load_tensor(st, name, it.shape, it.dst, it.dt, stream))) return bail("");
        }
    }
    anelm_st_close(st);
    st = nullptr;
    ALLOC(m->cos_tab, float, (long)kRopeRows * (D / 2));
    ALLOC(m->sin_tab, float, (long)kRopeRows * (D / 2));
    const long amax = std::max({H, (long)m->qdim, I});
    ALLOC(m->x, float, B * H);
    ALLOC(m->xn, float, B * H);
    ALLOC(m->qkv, float, B * m->qkvdim);
    ALLOC(m->attn, float, B * m->qdim);
    ALLOC(m->o, float, B * H);
    ALLOC(m->gu, float, B * 2 * I);
    ALLOC(m->h, float, B * I);
    const long Bp = (B + 15) / 16 * 16;   // whole 16-row tiles for the tiled activations
    ALLOC(m->a16, uint16_t, Bp * amax);
    ALLOC(m->y16, uint16_t, Bp * std::max({(long)m->qkvdim, 2 * I, H}));
#undef ALLOC
    // Past 16 sequences the LM head streams a tiled copy of its W (1 KB per
    // load instruction) through the LDS kernel; made once here.
    if (B > 16 && c.hidden % 256 == 0 && c.hidden <= 4096 && c.vocab >= 8192) {
        const size_t tb = anelm_proj_tiled_size(c.vocab, c.hidden);
        if (!(m->lm_tiled = static_cast<uint16_t*>(m->alloc(tb)))) {
            rc = fail(ANELM_ERR_HIP, "qwen3_load: out of device memory");
            delete m;
            return nullptr;
        }
        if ((rc = anelm_proj_tile_f16(m->lm_tiled, m->lm16, c.vocab, c.hidden, stream))) {
            delete m;
            return nullptr;
        }
    }
    // Past 16 sequences the layer projections read tiled copies too (each
    // weight load instruction 1 KB in a row; the row-major weights stay for
    // steps of up to 16 sequences), and their fp16 inputs are tiled as well
    if (B > 16 && H % 32 == 0 && I % 32 == 0 && m->qdim % 32 == 0) {
        for (anelm_qwen3::Layer& l : m->layers) {
            struct Tile {
                uint16_t** dst;
                const uint16_t* src;
                long rows, cols;
            } tiles[] = {{&l.qkv_t, l.qkv16, m->qkvdim, H}, {&l.o_t, l.o16, H, m->qdim},
                         {&l.gu_t, l.gu16, 2 * I, H}, {&l.down_t, l.down16, H, I}};
            for (const Tile& t : tiles) {
                const size_t tb = anelm_proj_tiled_size((int)t.rows, (int)t.cols);
                if (!(*t.dst = static_cast<uint16_t*>(m->alloc(tb)))) {
                    rc = fail(ANELM_ERR_HIP, "qwen3_load: out of device memory");
                    delete m;
                    return nullptr;
                }
                if ((rc = anelm_proj_tile_f16(*t.dst, t.src, (int)t.rows, (int)t.cols, stream))) {
                    delete m;
                    return nullptr;
                }
            }
        }
    }
    m->attn_ws_bytes = anelm_gqa_workspace_size(B, c.n_q_heads, c.n_kv_heads, c.head_dim, m->cap);
    if (m->attn_ws_bytes && (!(m->attn_ws = m->alloc(m->attn_ws_bytes)) ||
                             hipMemsetAsync(m->attn_ws, 0, m->attn_ws_bytes, anelm::as_stream(stream)) != hipSuccess)) {
        // the attention's workspace starts zero-filled; each call leaves it so
        rc = fail(ANELM_ERR_HIP, "qwen3_load: out of device memory");
        delete m;
        return nullptr;
    }
    if ((rc = anelm_rope_table(m->cos_tab, m->sin_tab, kRopeRows, c.head_dim, c.rope_theta, stream)) ||
        (rc = anelm_qwen3_reset(m, stream))) {
        delete m;
        return nullptr;
    }
    if (hipStreamSynchronize(anelm::as_stream(stream)) != hipSuccess) {
        fail(ANELM_ERR_HIP, "qwen3_load: synchronisation failed");
        delete m;
        return nullptr;
    }
    return m;
}

extern "C" void anelm_qwen3_free(anelm_qwen3* m) { delete m; }

extern "C" int anelm_qwen3_reset(anelm_qwen3* m, void* stream) {
    clear_error();
    if (!m) return fail(ANELM_ERR_INVALID, "qwen3_reset: null model");
    const size_t n = sizeof(int32_t) * m->layers.size() * m->max_batch;
    if (hipMemsetAsync(m->ring_start, 0, n, anelm::as_stream(stream)) != hipSuccess ||
        hipMemsetAsync(m->ring_len, 0, n, anelm::as_stream(stream)) != hipSuccess)
        return fail(ANELM_ERR_HIP, "qwen3_reset: hipMemsetAsync failed");
    return ANELM_OK;
}

// models/llm/qwen3.cpp:497-564 for `batch` sequences, one token each.
extern "C" int anelm_qwen3_forward(anelm_qwen3* m, const int32_t* ids, const int32_t* pos, long batch,
                                   float* logits, long ld_logits, int32_t* bad_ids, void* stream) {
    clear_error();
    if (!m || !ids || !pos || !logits) return fail(ANELM_ERR_INVALID, "qwen3_forward: null pointer");
    const anelm_qwen3_config& c = m->c;
    if (batch <= 0 || batch > m->max_batch || ld_logits < c.vocab)
        return fail(ANELM_ERR_INVALID, "qwen3_forward: batch %ld (max %d) or ld_logits", batch, m->max_batch);
    const long H = c.hidden, I = c.intermediate, V = c.vocab, B = batch;
    const long seq = (long)m->cap * m->kvdim;
    int rc;
#define CK(call)                      \
    do {                              \
        if ((rc = (call)) != ANELM_OK) return rc; \
    } while (0)
    // out = the fp16 projection of the [B, n_in] fp32 rows, widened: MFMA
    // kernels for in_dim a multiple of 32 (past 16 rows from inputs rounded
    // to fp16 once), else the dot kernel up to 8 rows and the any-shape
    // kernel beyond (dims no Qwen3 size has)
    auto project = [&](float* out, long ld_out, const float* in, long n_in, const uint16_t* w16, long n_out) -> int {
        int r;
        if (n_in % 32 == 0 && B > 16) {
            if ((r = anelm_f32_to_f16(m->a16, in, (size_t)(B * n_in), stream))) return r;
            return anelm_proj_f16_x16(out, m->a16, w16, B, (int)n_out, (int)n_in, n_in, ld_out, stream);
        }
        return anelm_proj_f16(out, in, w16, B, (int)n_out, (int)n_in, n_in, ld_out, stream);
    };
    // q/k norm + RoPE, the KV ring append and the attention, one launch
    // (head_dim 128) over the raw q|k|v rows; every layer's rings were
    // advanced at the start of the step
    auto attend = [&](const anelm_qwen3::Layer& l, void* out, int out_f16) -> int {
        return anelm_gqa_attention_qk(out, out_f16, m->qkv, m->qkv + m->qdim, m->qkv + m->qdim + m->kvdim, m->qkvdim,
                                      m->qkvdim, m->qkvdim, l.qn, l.kn, ANELM_BF16, pos, m->cos_tab, m->sin_tab,
                                      kRopeRows, c.rope_theta, c.rms_eps, l.kc, l.vc, l.start, l.len, B, c.n_q_heads,
                                      c.n_kv_heads, m->qdim, m->cap, seq, m->attn_ws, m->attn_ws_bytes, stream);
    };
    CK(anelm_embed_gather(m->x, m->embed, ANELM_BF16, ids, B, H, V, bad_ids, stream));             // :498
    CK(anelm_kv_ring_advance(m->ring_start, m->ring_len, B, c.layers, m->max_batch, m->cap, stream));  // :475-484
    const bool dims32 = H % 32 == 0 && I % 32 == 0 && m->qdim % 32 == 0;
    if (dims32 && B > 16) {
        // Past 16 rows every projection input is fp16 in the tiled layout
        // (16 rows x 32 columns per contiguous 1 KB piece), as are the
        // weights (made at load): the RMSNorms round their output to fp16
        // once, the attention writes the o projection's input and the SwiGLU
        // the down projection's; the residual adds ride in the o and down
        // projections.  7 calls per layer.
        if (!m->layers.empty() && !m->layers[0].qkv_t) return fail(ANELM_ERR_INVALID, "qwen3_forward: no tiled weights");
        for (int L = 0; L < c.layers; L++) {
            const anelm_qwen3::Layer& l = m->layers[L];
            CK(anelm_rmsnorm_f16_tiled(m->a16, m->x, l.w_in, ANELM_BF16, B, (int)H, H, c.rms_eps, stream));  // :503
            CK(anelm_proj_f16_tt(m->qkv, m->a16, l.qkv_t, B, m->qkvdim, (int)H, m->qkvdim, ANELM_PROJ_STORE,
                                 stream));                                                        // first_proj
            CK(attend(l, m->y16, 2));                                                             // :444-490
            CK(anelm_proj_f16_tt(m->x, m->y16, l.o_t, B, (int)H, m->qdim, H, ANELM_PROJ_ADD, stream));  // o_proj + :516
            CK(anelm_rmsnorm_f16_tiled(m->a16, m->x, l.w_post, ANELM_BF16, B, (int)H, H, c.rms_eps, stream));  // :518
            CK(anelm_proj_f16_tt(m->y16, m->a16, l.gu_t, B, (int)I, (int)H, I, ANELM_PROJ_SWIGLU_F16_TILED,
                                 stream));                                                        // fused_ffn
            CK(anelm_proj_f16_tt(m->x, m->y16, l.down_t, B, (int)H, (int)I, H, ANELM_PROJ_ADD, stream));  // down + :527
        }
        CK(anelm_rmsnorm_f16(m->a16, m->x, m->final_norm, ANELM_BF16, B, (int)H, H, H, c.rms_eps, stream));  // :530
        // the LM head (a 151936-row W streams once through the LDS-staged
        // kernel, from its tiled copy) writes the widened logits itself
        if (m->lm_tiled)
            return anelm_proj_f16_x16_tiled(logits, m->a16, m->lm_tiled, B, (int)V, (int)H, H, ld_logits,
                                            ANELM_PROJ_STORE, stream);
        return anelm_proj_f16_x16_fused(logits, m->a16, m->lm16, B, (int)V, (int)H, H, ld_logits, ANELM_PROJ_STORE,
                                        stream);
    }
    if (dims32) {
        // 5 calls per layer: the RMSNorms, residual adds and the SwiGLU
        // ride in the projections; the attention and the SwiGLU hand the o
        // and down projections their inputs already rounded to fp16 (the
        // rounding those projections apply to their inputs anyway)
        for (int L = 0; L < c.layers; L++) {
            const anelm_qwen3::Layer& l = m->layers[L];
            CK(anelm_proj_f16_fused(m->qkv, m->x, l.qkv16, B, m->qkvdim, (int)H, H, m->qkvdim, l.w_in, c.rms_eps,
                                    ANELM_PROJ_STORE, stream));                                   // :503 + first_proj
            CK(attend(l, m->y16, 1));                                                             // :444-490
            CK(anelm_proj_f16_x16_fused(m->x, m->y16, l.o16, B, (int)H, m->qdim, m->qdim, H, ANELM_PROJ_ADD,
                                        stream));                                                 // o_proj + :516
            CK(anelm_proj_f16_fused(m->y16, m->x, l.gu16, B, (int)I, (int)H, H, I, l.w_post, c.rms_eps,
                                    ANELM_PROJ_SWIGLU_F16, stream));                              // :518 + fused_ffn
            CK(anelm_proj_f16_x16_fused(m->x, m->y16, l.down16, B, (int)H, (int)I, I, H, ANELM_PROJ_ADD,
                                        stream));                                                 // down + :527
        }
        CK(anelm_proj_f16_fused(logits, m->x, m->lm16, B, (int)V, (int)H, H, ld_logits, m->final_norm, c.rms_eps,
                                ANELM_PROJ_STORE, stream));                                       // :530 + LM head
        return ANELM_OK;
    }
    for (int L = 0; L < c.layers; L++) {
        const anelm_qwen3::Layer& l = m->layers[L];
        CK(anelm_rmsnorm(m->xn, m->x, l.w_in, ANELM_BF16, B, (int)H, H, H, c.rms_eps, stream));    // :503
        CK(project(m->qkv, m->qkvdim, m->xn, H, l.qkv16, m->qkvdim));                             // first_proj
        CK(attend(l, m->attn, 0));                                                                // :444-490
        CK(project(m->o, H, m->attn, m->qdim, l.o16, H));                                         // o_proj
        CK(anelm_add_rmsnorm(m->x, m->o, m->xn, l.w_post, ANELM_BF16, B, (int)H, H, H, H, c.rms_eps,
                             stream));                                                            // :516-518
        CK(project(m->gu, 2 * I, m->xn, H, l.gu16, 2 * I));                                       // fused_ffn: gate|up
        CK(anelm_silu_mul(m->h, m->gu, m->gu + I, B, I, I, 2 * I, 2 * I, stream));
        CK(project(m->o, H, m->h, I, l.down16, H));                                               // fused_ffn: down
        CK(anelm_residual_add(m->x, m->o, (size_t)(B * H), stream));                             // :527
    }
    CK(anelm_rmsnorm(m->x, m->x, m->final_norm, ANELM_BF16, B, (int)H, H, H, c.rms_eps, stream));  // :530
    CK(project(logits, ld_logits, m->x, H, m->lm16, V));                                          // LM head
#undef CK
    return ANELM_OK;
}
