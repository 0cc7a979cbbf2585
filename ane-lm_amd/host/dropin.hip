// The reference-signature drop-in layer (ane_lm::rmsnorm, ane_lm::softmax,
// ane_lm::sample_token, ...) over the C ABI.  Host pointers in, host pointers
// out: each call leases a staging slot (stream, pinned host buffer, device
// buffer) from a process-wide pool, runs the HIP kernels on the slot's
// stream and has the results in the caller's memory before returning, so
// callers that run these functions concurrently from several threads (as
// models/llm/qwen3.cpp:451-461 does) never share state.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "anelm_hip.h"
#include "ane_lm/convert.h"
#include "ane_lm/cpu_ops.h"
#include "ane_lm/sampling.h"

namespace ane_lm {
namespace {

[[noreturn]] void die(const char* what, const char* msg) {
    fprintf(stderr, "ane_lm (HIP): %s failed: %s\n", what, msg);
    abort();
}

void check_rc(int rc, const char* what) {
    if (rc != ANELM_OK) die(what, anelm_last_error());
}

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) die(what, hipGetErrorString(e));
}

// A staging slot: one HIP stream, a growable device buffer and a fixed
// pinned host buffer.  Slots are leased to one call at a time from a
// process-wide pool, so concurrent callers never share one, threads that
// come and go reuse them, and the pool holds as many as were ever in use at
// once.  Slots live until the process ends: the HIP runtime may already be
// shut down when static destructors run, and the pinned buffers, once read
// by kernels, are never returned.
constexpr size_t kPinBytes = (size_t)1 << 20;       // per slot
constexpr size_t kZeroCopyBytes = (size_t)512 << 10;  // operands the kernels read and write in host memory

struct Slot {
    hipStream_t stream = nullptr;
    char* dev = nullptr;
    size_t dev_cap = 0;
    char* pin = nullptr;   // kPinBytes of pinned, coherent host memory: zero-copy operands, or a staging image
};

std::mutex g_pool_mu;
std::vector<Slot*>* g_pool = new std::vector<Slot*>();

Slot* acquire_slot() {
    {
        std::lock_guard<std::mutex> lk(g_pool_mu);
        if (!g_pool->empty()) {
            Slot* s = g_pool->back();
            g_pool->pop_back();
            return s;
        }
    }
    Slot* s = new Slot();
    check_hip(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipHostMalloc(reinterpret_cast<void**>(&s->pin), kPinBytes, hipHostMallocCoherent), "hipHostMalloc");
    return s;
}

void release_slot(Slot* s) {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    g_pool->push_back(s);
}

// One call's lease on a slot.  get() places the call's operands: in the
// slot's pinned host buffer when they fit (the kernels then read and write
// them in host memory, and h2d/d2h are host copies before the launch and
// after the sync), else in device memory (h2d/d2h are stream copies).
// Workspace asked for in get() is always device memory.
class Lease {
  public:
    Lease() : slot_(acquire_slot()) {}
    ~Lease() { release_slot(slot_); }
    Lease(const Lease&) = delete;
    Lease& operator=(const Lease&) = delete;

    hipStream_t s() const { return slot_->stream; }

    template <size_t N>
    void get(const size_t (&sizes)[N], char* (&out)[N], size_t scratch = 0, char** scratch_out = nullptr) {
        size_t off[N], total = 0;
        for (size_t i = 0; i < N; i++) {
            off[i] = total;
            total += (sizes[i] + 255) & ~(size_t)255;
        }
        zero_copy_ = total <= kZeroCopyBytes;
        device((zero_copy_ ? 0 : total) + scratch);
        char* base = zero_copy_ ? slot_->pin : slot_->dev;
        for (size_t i = 0; i < N; i++) out[i] = base + off[i];
        if (scratch_out) *scratch_out = slot_->dev + (zero_copy_ ? 0 : total);
    }
    // The slot's device buffer, at least n bytes.
    char* device(size_t n) {
        if (n > slot_->dev_cap) {
            if (slot_->dev) check_hip(hipFree(slot_->dev), "hipFree");
            const size_t ncap = n < ((size_t)1 << 20) ? ((size_t)1 << 20) : n;
            check_hip(hipMalloc(reinterpret_cast<void**>(&slot_->dev), ncap), "hipMalloc");
            slot_->dev_cap = ncap;
        }
        return slot_->dev;
    }
    // The slot's pinned buffer (kPinBytes), for a call that lays out its own
    // staging image; the call's sync() orders its reuse.
    char* pinned() const { return slot_->pin; }
    // One copy of the first n bytes of the pinned buffer to d.
    void h2d_staged(void* d, size_t n) {
        check_hip(hipMemcpyAsync(d, slot_->pin, n, hipMemcpyHostToDevice, s()), "hipMemcpy H2D");
    }
    void h2d(void* d, const void* h, size_t n) {
        if (zero_copy_)
            std::memcpy(d, h, n);
        else
            check_hip(hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, s()), "hipMemcpy H2D");
    }
    void d2h(void* h, const void* d, size_t n) {
        if (!zero_copy_) {
            check_hip(hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, s()), "hipMemcpy D2H");
            return;
        }
        if (nout_ == kMaxOut) die("drop-in staging", "too many outputs");
        outs_[nout_++] = {h, d, n};
    }
    // Waits for the call's work, then copies zero-copy outputs out.
    void sync() {
        check_hip(hipStreamSynchronize(s()), "hipStreamSynchronize");
        for (int i = 0; i < nout_; i++) std::memcpy(outs_[i].h, outs_[i].d, outs_[i].n);
        nout_ = 0;
    }

  private:
    static constexpr int kMaxOut = 8;
    struct Out {
        void* h;
        const void* d;
        size_t n;
    };
    Slot* slot_;
    bool zero_copy_ = false;
    Out outs_[kMaxOut];
    int nout_ = 0;
};

}  // namespace

// core/cpu_ops.cpp:7-14
void silu_vec_inplace(float* x, int n, float* /*tmp*/) {
    if (n <= 0) return;
    Lease S;
    const size_t sz[1] = {(size_t)n * 4};
    char* d[1];
    S.get(sz, d);
    S.h2d(d[0], x, sz[0]);
    check_rc(anelm_silu(reinterpret_cast<float*>(d[0]), (size_t)n, S.s()), "silu_vec_inplace");
    S.d2h(x, d[0], sz[0]);
    S.sync();
}

// core/cpu_ops.cpp:16-23
void mul_sigmoid_inplace(float* y, const float* z, int n, float* /*tmp*/) {
    if (n <= 0) return;
    Lease S;
    const size_t sz[2] = {(size_t)n * 4, (size_t)n * 4};
    char* d[2];
    S.get(sz, d);
    S.h2d(d[0], y, sz[0]);
    S.h2d(d[1], z, sz[1]);
    check_rc(anelm_mul_sigmoid(reinterpret_cast<float*>(d[0]), reinterpret_cast<const float*>(d[1]), (size_t)n, S.s()),
             "mul_sigmoid_inplace");
    S.d2h(y, d[0], sz[0]);
    S.sync();
}

// core/cpu_ops.cpp:25-31
void rmsnorm(float* out, const float* x, const float* weight, int dim, float eps) {
    if (dim <= 0) return;
    Lease S;
    const size_t sz[2] = {(size_t)dim * 4, (size_t)dim * 4};
    char* d[2];
    S.get(sz, d);
    S.h2d(d[0], x, sz[0]);
    S.h2d(d[1], weight, sz[1]);
    float* dx = reinterpret_cast<float*>(d[0]);
    check_rc(anelm_rmsnorm(dx, dx, d[1], ANELM_F32, 1, dim, dim, dim, eps, S.s()), "rmsnorm");
    S.d2h(out, d[0], sz[0]);
    S.sync();
}

// core/cpu_ops.cpp:56-80
void apply_rope_cached(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim, int q_head_stride,
                       int k_head_stride, int rot_dim, int pos, float theta, const float* cos_row,
                       const float* sin_row) {
    const int nh = n_q_heads + n_kv_heads;
    if (nh <= 0 || rot_dim <= 0) return;
    Lease S;
    // span of each operand that the rotation touches
    const size_t qn = n_q_heads > 0 ? (size_t)(n_q_heads - 1) * q_head_stride + rot_dim : 0;
    const size_t kn = n_kv_heads > 0 ? (size_t)(n_kv_heads - 1) * k_head_stride + rot_dim : 0;
    const bool tab = cos_row && sin_row;
    const size_t half = (size_t)rot_dim / 2;
    const size_t sz[4] = {qn * 4, kn * 4, tab ? half * 4 : 0, tab ? half * 4 : 0};
    char* d[4];
    S.get(sz, d);
    if (qn) S.h2d(d[0], q, sz[0]);
    if (kn) S.h2d(d[1], k, sz[1]);
    if (tab) {
        S.h2d(d[2], cos_row, sz[2]);
        S.h2d(d[3], sin_row, sz[3]);
    }
    check_rc(anelm_rope_cached(qn ? reinterpret_cast<float*>(d[0]) : nullptr, kn ? reinterpret_cast<float*>(d[1]) : nullptr,
                               n_q_heads, n_kv_heads, head_dim, q_head_stride, k_head_stride, rot_dim, pos, theta,
                               tab ? reinterpret_cast<const float*>(d[2]) : nullptr,
                               tab ? reinterpret_cast<const float*>(d[3]) : nullptr, S.s()),
             "apply_rope_cached");
    if (qn) S.d2h(q, d[0], sz[0]);
    if (kn) S.d2h(k, d[1], sz[1]);
    S.sync();
}

// core/cpu_ops.cpp:83-99
void softmax(float* x, int n) {
    if (n <= 0) return;
    Lease S;
    const size_t ws = anelm_softmax_workspace_size(1, n);
    const size_t sz[1] = {(size_t)n * 4};
    char* d[1];
    char* dws = nullptr;
    S.get(sz, d, ws, &dws);
    S.h2d(d[0], x, sz[0]);
    check_rc(anelm_softmax(reinterpret_cast<float*>(d[0]), 1, n, n, dws, ws, S.s()), "softmax");
    S.d2h(x, d[0], sz[0]);
    S.sync();
}

// core/cpu_ops.cpp:33-39
void rmsnorm_gated(float* out, const float* x, const float* z, const float* weight, int dim) {
    if (dim <= 0) return;
    Lease S;
    const size_t n = (size_t)dim * 4;
    const size_t sz[4] = {n, n, n, n};
    char* d[4];
    S.get(sz, d);
    S.h2d(d[0], x, n);
    S.h2d(d[1], z, n);
    S.h2d(d[2], weight, n);
    check_rc(anelm_rmsnorm_gated(reinterpret_cast<float*>(d[3]), reinterpret_cast<const float*>(d[0]),
                                 reinterpret_cast<const float*>(d[1]), d[2], ANELM_F32, 1, 1, dim, dim, dim, dim,
                                 1e-6f, S.s()),
             "rmsnorm_gated");
    S.d2h(out, d[3], n);
    S.sync();
}

// core/cpu_ops.cpp:100-103
void matvec(float* y, const float* W, const float* x, int out_dim, int in_dim) {
    if (out_dim <= 0 || in_dim <= 0) return;
    Lease S;
    const size_t sz[3] = {(size_t)out_dim * in_dim * 4, (size_t)in_dim * 4, (size_t)out_dim * 4};
    char* d[3];
    S.get(sz, d);
    S.h2d(d[0], W, sz[0]);
    S.h2d(d[1], x, sz[1]);
    check_rc(anelm_matvec(reinterpret_cast<float*>(d[2]), reinterpret_cast<const float*>(d[0]),
                          reinterpret_cast<const float*>(d[1]), out_dim, in_dim, S.s()),
             "matvec");
    S.d2h(y, d[2], sz[2]);
    S.sync();
}

// core/cpu_ops.cpp:105-110
void l2_normalize(float* x, int dim) {
    if (dim <= 0) return;
    Lease S;
    const size_t sz[1] = {(size_t)dim * 4};
    char* d[1];
    S.get(sz, d);
    S.h2d(d[0], x, sz[0]);
    check_rc(anelm_l2_normalize(reinterpret_cast<float*>(d[0]), 1, 1, dim, dim, 1.0f, S.s()), "l2_normalize");
    S.d2h(x, d[0], sz[0]);
    S.sync();
}

// core/cpu_ops.cpp:112-150
void conv1d_update(float* y, float* conv_state, int* state_pos, const float* x, const float* w, int channels,
                   int kernel_size) {
    if (channels <= 0 || kernel_size < 2) return;
    Lease S;
    const size_t sn = (size_t)channels * (kernel_size - 1) * 4;
    const size_t sz[5] = {(size_t)channels * 4, sn, 4, (size_t)channels * 4, (size_t)channels * kernel_size * 4};
    char* d[5];
    S.get(sz, d);
    const int32_t pos = *state_pos;
    S.h2d(d[1], conv_state, sn);
    S.h2d(d[2], &pos, 4);
    S.h2d(d[3], x, sz[3]);
    S.h2d(d[4], w, sz[4]);
    check_rc(anelm_conv1d_update(reinterpret_cast<float*>(d[0]), reinterpret_cast<float*>(d[1]),
                                 reinterpret_cast<int32_t*>(d[2]), reinterpret_cast<const float*>(d[3]),
                                 reinterpret_cast<const float*>(d[4]), 1, channels, kernel_size, channels, channels,
                                 (long)channels * (kernel_size - 1), S.s()),
             "conv1d_update");
    int32_t npos = 0;
    S.d2h(y, d[0], sz[0]);
    S.d2h(conv_state, d[1], sn);
    S.d2h(&npos, d[2], 4);
    S.sync();
    *state_pos = npos;
}

// core/cpu_ops.cpp:152-171
void ssm_step(float* y, float* state, const float* q, const float* k, const float* v, float decay, float beta,
              int key_dim, int value_dim) {
    Lease S;
    const size_t sn = (size_t)key_dim * value_dim * 4;
    const size_t sz[7] = {(size_t)value_dim * 4, sn, (size_t)key_dim * 4, (size_t)key_dim * 4,
                          (size_t)value_dim * 4, 4, 4};
    char* d[7];
    S.get(sz, d);
    S.h2d(d[1], state, sn);
    S.h2d(d[2], q, sz[2]);
    S.h2d(d[3], k, sz[3]);
    S.h2d(d[4], v, sz[4]);
    S.h2d(d[5], &decay, 4);
    S.h2d(d[6], &beta, 4);
    check_rc(anelm_ssm_step(reinterpret_cast<float*>(d[0]), reinterpret_cast<float*>(d[1]),
                            reinterpret_cast<const float*>(d[2]), reinterpret_cast<const float*>(d[3]),
                            reinterpret_cast<const float*>(d[4]), reinterpret_cast<const float*>(d[5]),
                            reinterpret_cast<const float*>(d[6]), 1, 1, 1, key_dim, value_dim, key_dim, value_dim,
                            value_dim, (long)key_dim * value_dim, S.s()),
             "ssm_step");
    S.d2h(y, d[0], sz[0]);
    S.d2h(state, d[1], sn);
    S.sync();
}

// core/cpu_ops.cpp:173-240
void gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache, int n_heads,
                   int n_kv_heads, int head_dim, int q_head_stride, int cache_start, int cache_len,
                   int cache_capacity) {
    if (n_heads <= 0 || head_dim <= 0) return;
    if (cache_len <= 0) {  // :177-180
        std::memset(out, 0, (size_t)n_heads * head_dim * sizeof(float));
        return;
    }
    Lease S;
    const size_t qn = (size_t)(n_heads - 1) * q_head_stride + head_dim;
    const size_t cn = (size_t)cache_capacity * n_kv_heads * head_dim;
    const size_t on = (size_t)n_heads * head_dim;
    const size_t ws = anelm_gqa_workspace_size(1, n_heads, n_kv_heads, head_dim, cache_capacity);
    const size_t sz[4] = {qn * 4, cn * 4, cn * 4, on * 4};
    char* d[4];
    char* dws = nullptr;
    S.get(sz, d, ws, &dws);
    // the attention's workspace starts zero-filled (pooled scratch holds
    // whatever the last call on this slot left)
    if (ws && hipMemsetAsync(dws, 0, ws, S.s()) != hipSuccess) die("gqa_attention", "hipMemsetAsync failed");
    S.h2d(d[0], q, sz[0]);
    S.h2d(d[1], k_cache, sz[1]);
    S.h2d(d[2], v_cache, sz[2]);
    check_rc(anelm_gqa_attention_ring(reinterpret_cast<float*>(d[3]), reinterpret_cast<const float*>(d[0]),
                                      reinterpret_cast<const float*>(d[1]), reinterpret_cast<const float*>(d[2]),
                                      n_heads, n_kv_heads, head_dim, q_head_stride, cache_start, cache_len,
                                      cache_capacity, ws ? dws : nullptr, ws, S.s()),
             "gqa_attention");
    S.d2h(out, d[3], sz[3]);
    S.sync();
}

// core/sampling.cpp:10-66
int sample_token(const float* logits, int vocab_size, const SamplingParams& params,
                 const std::vector<int>& recent_tokens) {
    if (vocab_size <= 0) die("sample_token", "vocab_size <= 0");
    Lease S;
    const long nh = (long)recent_tokens.size();
    const size_t ws = anelm_sample_workspace_size(1, vocab_size);
    const bool draw = params.temperature > 0.0f;
    // the reference's draw (sampling.cpp:58), only on the sampling path
    const float r = draw ? (float)drand48() : 0.0f;
    anelm_sampling_params p;
    p.temperature = params.temperature;
    p.repetition_penalty = params.repetition_penalty;
    p.repetition_context_size = params.repetition_context_size;
    p.frequency_penalty = params.frequency_penalty;
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const size_t lb = (size_t)vocab_size * 4, hb = (size_t)(nh > 0 ? nh : 1) * 4;
    const size_t o_hist = up(lb), o_r = o_hist + up(hb), in_bytes = o_r + 256;
    if (in_bytes + 256 <= kPinBytes) {
        // The inputs as one image in the pinned buffer, one copy to the
        // device (the vocabulary's logits are read by several kernels, so
        // they go to HBM once rather than over the bus per read); the id
        // comes back zero-copy behind the image, the probabilities (written,
        // never read back) and the workspace stay on the device.
        char* pin = S.pinned();
        char* dev = S.device(in_bytes + up(lb) + ws);
        std::memcpy(pin, logits, lb);
        if (nh > 0) std::memcpy(pin + o_hist, recent_tokens.data(), (size_t)nh * 4);
        std::memcpy(pin + o_r, &r, 4);
        volatile int32_t* id = reinterpret_cast<volatile int32_t*>(pin + in_bytes);
        S.h2d_staged(dev, in_bytes);
        check_rc(anelm_sample(const_cast<int32_t*>(id), reinterpret_cast<float*>(dev + in_bytes), vocab_size,
                              reinterpret_cast<const float*>(dev), vocab_size, 1, vocab_size,
                              nh > 0 ? reinterpret_cast<const int32_t*>(dev + o_hist) : nullptr, nh, nullptr, &p,
                              reinterpret_cast<const float*>(dev + o_r), ws ? dev + in_bytes + up(lb) : nullptr, ws,
                              S.s()),
                 "sample_token");
        S.sync();
        return *id;
    }
    // the probabilities (d[4]) are written and never read back
    const size_t sz[5] = {lb, hb, 16, 16, lb};
    char* d[5];
    char* dws = nullptr;
    S.get(sz, d, ws, &dws);
    S.h2d(d[0], logits, sz[0]);
    if (nh > 0) S.h2d(d[1], recent_tokens.data(), (size_t)nh * 4);
    S.h2d(d[2], &r, 4);
    check_rc(anelm_sample(reinterpret_cast<int32_t*>(d[3]), reinterpret_cast<float*>(d[4]), vocab_size,
                          reinterpret_cast<const float*>(d[0]),
                          vocab_size, 1, vocab_size, nh > 0 ? reinterpret_cast<const int32_t*>(d[1]) : nullptr, nh,
                          nullptr, &p, reinterpret_cast<const float*>(d[2]), dws, ws, S.s()),
             "sample_token");
    int32_t id = 0;
    S.d2h(&id, d[3], 4);
    S.sync();
    return id;
}

namespace hip {

void residual_add(float* x, const float* y, int n) {
    if (n <= 0) return;
    Lease S;
    const size_t sz[2] = {(size_t)n * 4, (size_t)n * 4};
    char* d[2];
    S.get(sz, d);
    S.h2d(d[0], x, sz[0]);
    S.h2d(d[1], y, sz[1]);
    check_rc(anelm_residual_add(reinterpret_cast<float*>(d[0]), reinterpret_cast<const float*>(d[1]), (size_t)n, S.s()),
             "residual_add");
    S.d2h(x, d[0], sz[0]);
    S.sync();
}

void qknorm_rope_qwen3(float* q, float* k, int nq, int nk, int head_dim, const float* q_norm, const float* k_norm,
                       float eps, int pos, float theta, const float* cos_row, const float* sin_row) {
    if (nq + nk <= 0 || head_dim <= 0) return;
    Lease S;
    const size_t qn = (size_t)nq * head_dim, kn = (size_t)nk * head_dim, half = (size_t)head_dim / 2;
    const bool tab = cos_row && sin_row;
    const size_t sz[7] = {qn * 4, kn * 4, (size_t)head_dim * 4, (size_t)head_dim * 4, half * 4, half * 4, 4};
    char* d[7];
    S.get(sz, d);
    if (qn) S.h2d(d[0], q, sz[0]);
    if (kn) S.h2d(d[1], k, sz[1]);
    if (q_norm) S.h2d(d[2], q_norm, sz[2]);
    if (k_norm) S.h2d(d[3], k_norm, sz[3]);
    if (tab) {
        S.h2d(d[4], cos_row, sz[4]);
        S.h2d(d[5], sin_row, sz[5]);
    }
    // with a table the row is passed as a one-row table at position 0
    const int32_t p = tab ? 0 : pos;
    S.h2d(d[6], &p, 4);
    check_rc(anelm_qknorm_rope(qn ? reinterpret_cast<float*>(d[0]) : nullptr, kn ? reinterpret_cast<float*>(d[1]) : nullptr,
                               (long)qn, (long)kn, q_norm ? d[2] : nullptr, k_norm ? d[3] : nullptr, ANELM_F32,
                               reinterpret_cast<const int32_t*>(d[6]), tab ? reinterpret_cast<const float*>(d[4]) : nullptr,
                               tab ? reinterpret_cast<const float*>(d[5]) : nullptr, tab ? 1 : 0, theta, 1, nq, nk, head_dim,
                               eps, S.s()),
             "qknorm_rope_qwen3");
    if (qn) S.d2h(q, d[0], sz[0]);
    if (kn) S.d2h(k, d[1], sz[1]);
    S.sync();
}

void silu_mul(float* h, const float* g, const float* u, int n) {
    if (n <= 0) return;
    Lease S;
    const size_t sz[2] = {(size_t)n * 4, (size_t)n * 4};
    char* d[2];
    S.get(sz, d);
    S.h2d(d[0], g, sz[0]);
    S.h2d(d[1], u, sz[1]);
    float* dg = reinterpret_cast<float*>(d[0]);
    check_rc(anelm_silu_mul(dg, dg, reinterpret_cast<const float*>(d[1]), 1, n, n, n, n, S.s()), "silu_mul");
    S.d2h(h, d[0], sz[0]);
    S.sync();
}

void bf16_to_f16_vec_n(uint16_t* out, const uint16_t* in, size_t n) {
    if (n == 0) return;
    Lease S;
    const size_t sz[1] = {n * 2};
    char* d[1];
    S.get(sz, d);
    S.h2d(d[0], in, sz[0]);
    uint16_t* dp = reinterpret_cast<uint16_t*>(d[0]);
    check_rc(anelm_bf16_to_f16(dp, dp, n, S.s()), "bf16_to_f16_vec");
    S.d2h(out, d[0], sz[0]);
    S.sync();
}

void bf16_to_f16_vec(uint16_t* out, const uint16_t* in, int n) {
    if (n > 0) bf16_to_f16_vec_n(out, in, (size_t)n);
}

}  // namespace hip
}  // namespace ane_lm
