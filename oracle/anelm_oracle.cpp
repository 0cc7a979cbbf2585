// anelm_oracle.cpp -- CPU restatement of the reference's fused layer-op path.
//
// TEST INFRASTRUCTURE ONLY: the checker for tests/, smoke() and the CPU
// baseline in bench.py.  Nothing in the product links or loads it.
//
// Built with -O3 -ffp-contract=off (no fast-math, IEEE denormals) so that
// every rounding step written below is the rounding step executed; the one
// fused multiply-add the reference's compiler forms (the frequency penalty,
// see orc_sample_token) is written as an explicit fmaf.
#include "anelm_oracle.h"

#include <cmath>
#include <cstring>
#include <cstdlib>
#include <map>
#include <vector>
#include <algorithm>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

static int nthreads_or_default(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

extern "C" int orc_max_threads(void) { return nthreads_or_default(0); }

// ---------------------------------------------------------------- converts
// include/ane_lm/common.h:21-26
extern "C" float orc_bf16_to_f32(uint16_t bf) { return u2f((uint32_t)bf << 16); }

// common.h:28-32 (truncation of the low half)
extern "C" uint16_t orc_f32_to_bf16(float f) { return (uint16_t)(f2u(f) >> 16); }

// common.h:35-56.  Subnormals: mant/1024 * 2^-14 (both steps exact);
// exponent 31 keeps the NaN payload bits (no quieting).
extern "C" float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float f = (float)m / 1024.0f;
        f *= (1.0f / 16384.0f);
        return sign ? -f : f;
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

// common.h:58-71.  Truncating (round toward zero) narrowing; exponent
// overflow and NaN both give +-Inf; below 2^-25 gives +-0.
extern "C" uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int32_t e = (int32_t)((u >> 23) & 0xFFu) - 127 + 15;
    uint32_t m = u & 0x7FFFFFu;
    if (e <= 0) {
        if (e < -10) return sign;
        m = (m | 0x800000u) >> (1 - e);
        return (uint16_t)(sign | (uint16_t)(m >> 13));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)(e << 10) | (uint16_t)(m >> 13));
}

// common.h:73-75
extern "C" uint16_t orc_bf16_to_f16(uint16_t bf) { return orc_f32_to_f16(orc_bf16_to_f32(bf)); }

// common.h:81-83 (n widened to size_t)
extern "C" void orc_bf16_to_f16_vec(uint16_t* out, const uint16_t* in, size_t n, int nthreads) {
    int nt = nthreads_or_default(nthreads);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long i = 0; i < (long)n; i++) out[i] = orc_bf16_to_f16(in[i]);
}

// common.h:77-79
extern "C" void orc_bf16_to_f32_vec(float* out, const uint16_t* in, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

extern "C" void orc_f16_to_f32_vec(float* out, const uint16_t* in, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

// core/safetensors.cpp:299-306: widen, then the (1+w) offset over the first
// expected_numel entries
extern "C" void orc_norm_weight_vec(float* out, const uint16_t* in, size_t n, long expected_numel) {
    orc_bf16_to_f32_vec(out, in, n);
    for (long i = 0; i < expected_numel && (size_t)i < n; i++) out[i] += 1.0f;
}

// ---------------------------------------------------------------- RMSNorm
// core/cpu_ops.cpp:25-31:
//   vDSP_svesq(x, &ss)            ss = sum x^2
//   ss = 1.0f / sqrtf(ss/dim+eps) true divide and sqrt, not rsqrt
//   vDSP_vsmul(x, ss, out)        out = x * s   (rounded)
//   vDSP_vmul(out, weight, out)   out = out * w (rounded)
extern "C" void orc_rmsnorm(float* out, const float* x, const float* w, int dim, float eps) {
    double acc = 0.0;
    for (int i = 0; i < dim; i++) acc += (double)x[i] * (double)x[i];
    float ss = (float)acc;
    ss = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; i++) {
        float t = x[i] * ss;
        out[i] = t * w[i];
    }
}

extern "C" void orc_rmsnorm_rows(float* out, const float* x, const float* w, long rows, int dim,
                                 long ld_x, long ld_out, float eps, int nthreads) {
    int nt = nthreads_or_default(nthreads);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long r = 0; r < rows; r++) orc_rmsnorm(out + r * ld_out, x + r * ld_x, w, dim, eps);
}

// ---------------------------------------------------------------- activations
// core/cpu_ops.cpp:7-14: tmp = -x; tmp = exp(tmp); tmp += 1; x = x / tmp
extern "C" void orc_silu_vec(float* x, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float t = expf(-x[i]);
        t = t + 1.0f;
        x[i] = x[i] / t;
    }
}

// core/cpu_ops.cpp:16-23: tmp = -z; exp; += 1; y = y / tmp
extern "C" void orc_mul_sigmoid(float* y, const float* z, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float t = expf(-z[i]);
        t = t + 1.0f;
        y[i] = y[i] / t;
    }
}

// SwiGLU: silu(gate) * up (core/ane_runtime.cpp:393-395 order; fp32 silu in
// the cpu_ops.cpp:7-14 form; the product is one fp32 multiply).
extern "C" void orc_silu_mul(float* h, const float* g, const float* u, size_t n, int nthreads) {
    int nt = nthreads_or_default(nthreads);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long i = 0; i < (long)n; i++) {
        float t = expf(-g[i]);
        t = t + 1.0f;
        float s = g[i] / t;
        h[i] = s * u[i];
    }
}

// ---------------------------------------------------------------- RoPE
// models/llm/qwen3.cpp:206-209
extern "C" void orc_rope_inv_freq(float* inv_freq, int rot_dim, float theta) {
    for (int j = 0, i = 0; i < rot_dim; i += 2, j++)
        inv_freq[j] = 1.0f / powf(theta, (float)i / (float)rot_dim);
}

// models/llm/qwen3.cpp:210-218: angle = pos * inv_freq[j] in fp32 (pos
// converted to float), then cosf / sinf.
extern "C" void orc_rope_table(float* cos_tab, float* sin_tab, int n_pos, int rot_dim,
                               float theta) {
    int half = rot_dim / 2;
    std::vector<float> inv((size_t)half);
    orc_rope_inv_freq(inv.data(), rot_dim, theta);
    for (int pos = 0; pos < n_pos; pos++) {
        for (int j = 0; j < half; j++) {
            float angle = (float)pos * inv[(size_t)j];
            cos_tab[(size_t)pos * half + j] = cosf(angle);
            sin_tab[(size_t)pos * half + j] = sinf(angle);
        }
    }
}

// qwen3.cpp:17-26 (table path, vDSP_vmmsb / vDSP_vmma, products rounded
// separately here) and qwen3.cpp:39-49 (fallback: same half-split pairing,
// angle from the same inv_freq formula).
static void rope_head_half_split(float* v, int half, int pos, float theta, int rot_dim,
                                 const float* cos_row, const float* sin_row) {
    if (cos_row && sin_row) {
        std::vector<float> tmp((size_t)half);
        for (int j = 0; j < half; j++) tmp[(size_t)j] = v[j] * cos_row[j] - v[j + half] * sin_row[j];
        for (int j = 0; j < half; j++) v[j + half] = v[j + half] * cos_row[j] + v[j] * sin_row[j];
        for (int j = 0; j < half; j++) v[j] = tmp[(size_t)j];
    } else {
        for (int i = 0; i < half; i++) {
            float freq = 1.0f / powf(theta, (float)(2 * i) / (float)rot_dim);
            float angle = (float)pos * freq;
            float c = cosf(angle), s = sinf(angle);
            float v0 = v[i], v1 = v[i + half];
            v[i] = v0 * c - v1 * s;
            v[i + half] = v1 * c + v0 * s;
        }
    }
}

// qwen3.cpp:28-52
extern "C" void orc_rope_qwen3(float* q, float* k, int nq, int nk, int head_dim, int pos,
                               float theta, const float* cos_row, const float* sin_row) {
    int half = head_dim / 2;
    for (int h = 0; h < nq + nk; h++) {
        float* v = (h < nq) ? q + (size_t)h * head_dim : k + (size_t)(h - nq) * head_dim;
        rope_head_half_split(v, half, pos, theta, head_dim, cos_row, sin_row);
    }
}

// core/cpu_ops.cpp:56-80
extern "C" void orc_rope_cached(float* q, float* k, int nq, int nk, int head_dim,
                                int q_head_stride, int k_head_stride, int rot_dim, int pos,
                                float theta, const float* cos_row, const float* sin_row) {
    (void)head_dim;
    int half = rot_dim / 2;
    for (int h = 0; h < nq + nk; h++) {
        float* v = (h < nq) ? q + (size_t)h * q_head_stride : k + (size_t)(h - nq) * k_head_stride;
        if (cos_row && sin_row) {
            rope_head_half_split(v, half, pos, theta, rot_dim, cos_row, sin_row);
        } else {
            // cpu_ops.cpp:68-77: adjacent pairs (v[i], v[i+1])
            for (int i = 0; i < rot_dim; i += 2) {
                float freq = 1.0f / powf(theta, (float)i / (float)rot_dim);
                float angle = (float)pos * freq;
                float c = cosf(angle), s = sinf(angle);
                float v0 = v[i], v1 = v[i + 1];
                v[i] = v0 * c - v1 * s;
                v[i + 1] = v0 * s + v1 * c;
            }
        }
    }
}

// qwen3.cpp:444-472 for T tokens: per-head rmsnorm (in place, shared gamma)
// then apply_rope_qwen3 with the row chosen as at :463-469.
extern "C" void orc_qknorm_rope(float* q, float* k, long q_ld, long k_ld, const float* wq,
                                const float* wk, const int32_t* pos, const float* cos_tab,
                                const float* sin_tab, int tab_len, float theta, long T, int nq,
                                int nk, int head_dim, float eps, int nthreads) {
    int nt = nthreads_or_default(nthreads);
    int half = head_dim / 2;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long t = 0; t < T; t++) {
        float* qt = q + t * q_ld;
        float* kt = k + t * k_ld;
        if (wq)
            for (int h = 0; h < nq; h++) orc_rmsnorm(qt + (size_t)h * head_dim, qt + (size_t)h * head_dim, wq, head_dim, eps);
        if (wk)
            for (int h = 0; h < nk; h++) orc_rmsnorm(kt + (size_t)h * head_dim, kt + (size_t)h * head_dim, wk, head_dim, eps);
        int p = pos[t];
        const float* cr = nullptr;
        const float* sr = nullptr;
        if (p >= 0 && p < tab_len && cos_tab && sin_tab) {
            cr = cos_tab + (size_t)p * half;
            sr = sin_tab + (size_t)p * half;
        }
        orc_rope_qwen3(qt, kt, nq, nk, head_dim, p, theta, cr, sr);
    }
}

// ---------------------------------------------------------------- residual
// qwen3.cpp:516 / :527  vDSP_vadd(x, y, x): one IEEE add per element
extern "C" void orc_residual_add(float* x, const float* y, size_t n, int nthreads) {
    int nt = nthreads_or_default(nthreads);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long i = 0; i < (long)n; i++) x[i] = x[i] + y[i];
}

// ---------------------------------------------------------------- gather
// qwen3.cpp:498 memcpy of row id (table expanded to fp32 at load,
// qwen3.cpp:255-256); for fp16/bf16 tables the exact widenings above.
extern "C" int orc_embed_gather(float* out, const void* table, int dtype, const int32_t* ids,
                                long n_ids, long hidden, long vocab) {
    for (long b = 0; b < n_ids; b++)
        if (ids[b] < 0 || ids[b] >= vocab) return -1;
    for (long b = 0; b < n_ids; b++) {
        size_t off = (size_t)ids[b] * (size_t)hidden;
        float* o = out + (size_t)b * hidden;
        if (dtype == 0) {
            std::memcpy(o, (const float*)table + off, (size_t)hidden * sizeof(float));
        } else if (dtype == 1) {
            orc_f16_to_f32_vec(o, (const uint16_t*)table + off, (size_t)hidden);
        } else {
            orc_bf16_to_f32_vec(o, (const uint16_t*)table + off, (size_t)hidden);
        }
    }
    return 0;
}

// ---------------------------------------------------------------- softmax
// exp with a fixed IEEE operation sequence (Cody & Waite two-constant
// argument reduction, "Software Manual for the Elementary Functions", 1980;
// degree-7 Taylor polynomial by Horner with fused multiply-adds; scaling
// by an exact power of two, split in two multiplies when the result is
// subnormal so it is rounded once).  Every step is a correctly rounded IEEE
// operation, so any IEEE machine with subnormals enabled reproduces it bit
// for bit.  Accuracy against fp64 exp is checked by the tests (<= 1 ulp).
static const float kLog2e = 0x1.715476p+0f;
static const float kC1 = 0x1.63p-1f;          // 0.693359375 (9 significant bits)
static const float kC2 = -0x1.bd0106p-13f;    // ln2 - kC1
static const float kP2 = 0x1p-1f, kP3 = 0x1.555556p-3f, kP4 = 0x1.555556p-5f;
static const float kP5 = 0x1.111112p-7f, kP6 = 0x1.6c16c2p-10f, kP7 = 0x1.a01a02p-13f;

static inline float pow2i(int k) { return u2f((uint32_t)(k + 127) << 23); }  // -126 <= k <= 127

extern "C" float orc_sampler_expf(float x) {
    if (x != x) return x;
    if (x < -104.0f) return 0.0f;
    if (x > 89.0f) return INFINITY;
    float kf = rintf(x * kLog2e);
    int k = (int)kf;
    float r = fmaf(-kf, kC1, x);
    r = fmaf(-kf, kC2, r);
    float p = kP7;
    p = fmaf(p, r, kP6);
    p = fmaf(p, r, kP5);
    p = fmaf(p, r, kP4);
    p = fmaf(p, r, kP3);
    p = fmaf(p, r, kP2);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    if (k < -126) return (p * pow2i(k + 64)) * pow2i(-64);
    if (k > 127) return (p * pow2i(k - 1)) * 2.0f;
    return p * pow2i(k);
}

// shift = 63 - ceil(log2 n): every term e*2^shift <= 2^shift and n terms
// sum to <= 2^63, so the accumulator cannot overflow.
extern "C" int orc_softmax_shift(long n) {
    int c = 0;
    while ((1L << c) < n) c++;
    return 63 - c;
}

// The sum of the exps as an exact integer sum of floor(e * 2^shift), then
// one rounding to float.  Integer addition is associative, so the GPU's
// reduction order cannot change the result.  Any NaN term makes it NaN.
static float fixed_point_sum(const float* e, long n) {
    int shift = orc_softmax_shift(n);
    float scale = ldexpf(1.0f, shift);
    uint64_t acc = 0;
    bool nan = false;
    for (long i = 0; i < n; i++) {
        float v = e[i];
        if (v >= 0.0f && v <= 1.0f) acc += (uint64_t)(v * scale);
        else nan = true;
    }
    if (nan) return NAN;
    return ldexpf((float)acc, -shift);
}

// core/cpu_ops.cpp:83-99
extern "C" void orc_softmax(float* x, int n) {
    float m = x[0];
    for (int i = 1; i < n; i++) m = fmaxf(m, x[i]);               // vDSP_maxv  :86
    float neg = -m;
    for (int i = 0; i < n; i++) x[i] = x[i] + neg;                 // vDSP_vsadd :89
    for (int i = 0; i < n; i++) x[i] = orc_sampler_expf(x[i]);     // vvexpf     :92
    float sum = fixed_point_sum(x, n);                             // vDSP_sve   :95
    float inv = 1.0f / sum;                                        //            :97
    for (int i = 0; i < n; i++) x[i] = x[i] * inv;                 // vDSP_vsmul :98
}

// ------------------------------------------------ Qwen3.5 linear attention

// core/cpu_ops.cpp:33-39
extern "C" void orc_rmsnorm_gated(float* out, const float* x, const float* z, const float* w, int dim) {
    orc_rmsnorm(out, x, w, dim, 1e-6f);                                      // :35 (default eps)
    for (int i = 0; i < dim; i++) out[i] = out[i] / (1.0f + expf(-z[i]));   // mul_sigmoid_inplace :37
    for (int i = 0; i < dim; i++) out[i] = out[i] * z[i];                   // vDSP_vmul :38
}

// core/cpu_ops.cpp:105-110
extern "C" void orc_l2_normalize(float* x, int dim) {
    double ss = 0.0;
    for (int i = 0; i < dim; i++) ss += (double)x[i] * (double)x[i];      // vDSP_svesq :107
    const float norm = 1.0f / sqrtf((float)ss + 1e-12f);                   // :108
    for (int i = 0; i < dim; i++) x[i] = x[i] * norm;                      // vDSP_vsmul :109
}

// core/cpu_ops.cpp:112-150 (the kernel_size 4 branch :117-133 is this loop unrolled)
extern "C" void orc_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x, const float* w,
                                  int channels, int kernel_size) {
    const int state_len = kernel_size - 1;
    int pos = *state_pos;
    for (int c = 0; c < channels; c++) {
        float* st = conv_state + (size_t)c * state_len;
        const float* wc = w + (size_t)c * kernel_size;
        float sum = 0.0f;
        for (int j = 0; j < state_len; j++) {
            int idx = pos + j;
            if (idx >= state_len) idx -= state_len;
            sum = fmaf(st[idx], wc[j], sum);
        }
        y[c] = fmaf(x[c], wc[state_len], sum);
        st[pos] = x[c];
    }
    pos++;
    if (pos == state_len) pos = 0;
    *state_pos = pos;
}

// core/cpu_ops.cpp:152-171
extern "C" void orc_ssm_step(float* y, float* state, const float* q, const float* k, const float* v, float decay,
                             float beta, int key_dim, int value_dim) {
    std::vector<float> delta(value_dim);
    for (int j = 0; j < value_dim; j++) {                       // Sk = state^T k   :154-155
        double sk = 0.0;
        for (int i = 0; i < key_dim; i++) sk += (double)state[(size_t)i * value_dim + j] * k[i];
        delta[j] = v[j] - (float)sk;                            // :158
    }
    for (int i = 0; i < key_dim; i++) {                         // sscal :160, sger :161-162
        for (int j = 0; j < value_dim; j++) {
            float& s = state[(size_t)i * value_dim + j];
            const float scaled = s * decay;
            s = (float)((double)scaled + (double)beta * (double)k[i] * (double)delta[j]);
        }
    }
    for (int j = 0; j < value_dim; j++) {                       // y = state^T q   :164-165
        double acc = 0.0;
        for (int i = 0; i < key_dim; i++) acc += (double)state[(size_t)i * value_dim + j] * q[i];
        y[j] = (float)acc;
    }
}

// core/cpu_ops.cpp:100-103
extern "C" void orc_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim) {
#pragma omp parallel for schedule(static) if (out_dim >= 1024)
    for (int r = 0; r < out_dim; r++) {
        const float* wr = W + (size_t)r * in_dim;
        double acc = 0.0;
        for (int c = 0; c < in_dim; c++) acc += (double)wr[c] * x[c];
        y[r] = (float)acc;
    }
}

// ------------------------------------------- ANE contractions, Qwen3 decode step

// Round-to-nearest-even fp32 -> fp16 (IEEE 754 binary16), in integers.
extern "C" uint16_t orc_f32_to_f16_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));  // NaN, quiet
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);                           // rounds to >= 2^16: Inf
    if (ax < 0x38800000u) {                                  // below 2^-14: fp16 subnormal or zero
        if (ax < 0x33000000u) return (uint16_t)sign;         // below 2^-25: rounds to zero (tie -> even 0)
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const int e = (int)(ax >> 23);                       // value = m * 2^(e-150)
        const int sh = 126 - e;                              // m >> sh = value / 2^-24
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((ax >> 13) - (112u << 10));                // rebias exponent, keep 10 mantissa bits
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

extern "C" void orc_linear_f16(uint16_t* y16, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim,
                               int in_dim) {
    std::vector<double> xd((size_t)in_dim);
    for (long b = 0; b < batch; b++) {
        for (int i = 0; i < in_dim; i++) xd[i] = orc_f16_to_f32(x16[(size_t)b * in_dim + i]);
#pragma omp parallel for schedule(static) if (out_dim >= 256)
        for (int o = 0; o < out_dim; o++) {
            const uint16_t* wr = w16 + (size_t)o * in_dim;
            double acc = 0.0;
            for (int i = 0; i < in_dim; i++) acc += xd[i] * (double)orc_f16_to_f32(wr[i]);
            y16[(size_t)b * out_dim + o] = orc_f32_to_f16_rne((float)acc);
        }
    }
}

namespace {
struct OrcQwen3 {
    orc_qwen3_config c;
    int batch, cap, qdim, kvdim, qkvdim;
    std::vector<float> embed, final_norm, cos_tab, sin_tab;
    std::vector<uint16_t> lm16;
    struct Layer {
        std::vector<uint16_t> qkv16, o16, gu16, down16;
        std::vector<float> qn, kn, w_in, w_post;
        std::vector<float> kc, vc;   // [batch][cap][kvdim]
        std::vector<int> start, len;
    };
    std::vector<Layer> layers;
};

std::vector<float> widen_bf16(const uint16_t* p, size_t n) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; i++) v[i] = orc_bf16_to_f32(p[i]);
    return v;
}

std::vector<uint16_t> to_f16(const uint16_t* bf16, size_t n) {
    std::vector<uint16_t> v(n);
    orc_bf16_to_f16_vec(v.data(), bf16, n, 0);
    return v;
}

// y = fp16 projection of the fp32 vector x (RNE in, fp16 out, widened)
void project(float* y, const float* x, const uint16_t* w16, int out_dim, int in_dim) {
    std::vector<uint16_t> x16((size_t)in_dim), y16((size_t)out_dim);
    for (int i = 0; i < in_dim; i++) x16[i] = orc_f32_to_f16_rne(x[i]);
    orc_linear_f16(y16.data(), x16.data(), w16, 1, out_dim, in_dim);
    for (int o = 0; o < out_dim; o++) y[o] = orc_f16_to_f32(y16[o]);
}
}  // namespace

extern "C" void* orc_qwen3_create(const orc_qwen3_config* c, int batch, int kv_capacity, const uint16_t* embed,
                                  const uint16_t* const* lt, const uint16_t* final_norm, const uint16_t* lm_head) {
    OrcQwen3* m = new OrcQwen3();
    m->c = *c;
    m->batch = batch;
    m->cap = kv_capacity;
    const int H = c->hidden, D = c->head_dim, I = c->intermediate;
    m->qdim = c->n_q_heads * D;
    m->kvdim = c->n_kv_heads * D;
    m->qkvdim = m->qdim + 2 * m->kvdim;
    m->embed = widen_bf16(embed, (size_t)c->vocab * H);                          // qwen3.cpp:255-256
    m->final_norm = widen_bf16(final_norm, (size_t)H);
    m->lm16 = to_f16(lm_head ? lm_head : embed, (size_t)c->vocab * H);          // tied: qwen3.cpp:259-260, :383
    const int tab = 16384;                                                       // min(max_pos, 16384), :201
    m->cos_tab.resize((size_t)tab * (D / 2));
    m->sin_tab.resize((size_t)tab * (D / 2));
    orc_rope_table(m->cos_tab.data(), m->sin_tab.data(), tab, D, c->rope_theta);
    m->layers.resize(c->layers);
    for (int L = 0; L < c->layers; L++) {
        const uint16_t* const* t = lt + 11 * L;
        OrcQwen3::Layer& l = m->layers[L];
        l.qkv16.resize((size_t)m->qkvdim * H);                                  // fused_3: [q | k | v]
        orc_bf16_to_f16_vec(l.qkv16.data(), t[0], (size_t)m->qdim * H, 0);
        orc_bf16_to_f16_vec(l.qkv16.data() + (size_t)m->qdim * H, t[1], (size_t)m->kvdim * H, 0);
        orc_bf16_to_f16_vec(l.qkv16.data() + (size_t)(m->qdim + m->kvdim) * H, t[2], (size_t)m->kvdim * H, 0);
        l.o16 = to_f16(t[3], (size_t)H * m->qdim);
        l.qn = widen_bf16(t[4], (size_t)D);
        l.kn = widen_bf16(t[5], (size_t)D);
        l.gu16.resize((size_t)2 * I * H);                                       // fused_ffn: gate, up
        orc_bf16_to_f16_vec(l.gu16.data(), t[6], (size_t)I * H, 0);
        orc_bf16_to_f16_vec(l.gu16.data() + (size_t)I * H, t[7], (size_t)I * H, 0);
        l.down16 = to_f16(t[8], (size_t)H * I);
        l.w_in = widen_bf16(t[9], (size_t)H);
        l.w_post = widen_bf16(t[10], (size_t)H);
        l.kc.assign((size_t)batch * kv_capacity * m->kvdim, 0.0f);
        l.vc.assign((size_t)batch * kv_capacity * m->kvdim, 0.0f);
        l.start.assign(batch, 0);
        l.len.assign(batch, 0);
    }
    return m;
}

// models/llm/qwen3.cpp:497-564 for each sequence b (ids[b] at position pos[b])
extern "C" void orc_qwen3_forward(void* mp, const int32_t* ids, const int32_t* pos, float* logits) {
    OrcQwen3* m = static_cast<OrcQwen3*>(mp);
    const orc_qwen3_config& c = m->c;
    const int H = c.hidden, D = c.head_dim, I = c.intermediate;
    std::vector<float> x(H), xn(H), qkv(m->qkvdim), attn(m->qdim), o(H), gu(2 * I), h(I);
    for (int b = 0; b < m->batch; b++) {
        std::memcpy(x.data(), m->embed.data() + (size_t)ids[b] * H, (size_t)H * 4);            // :498
        for (int L = 0; L < c.layers; L++) {
            OrcQwen3::Layer& l = m->layers[L];
            orc_rmsnorm(xn.data(), x.data(), l.w_in.data(), H, c.rms_eps);                    // :503
            project(qkv.data(), xn.data(), l.qkv16.data(), m->qkvdim, H);                     // first_proj
            orc_qknorm_rope(qkv.data(), qkv.data() + m->qdim, m->qkvdim, m->qkvdim, l.qn.data(), l.kn.data(),
                            &pos[b], m->cos_tab.data(), m->sin_tab.data(), 16384, c.rope_theta, 1,
                            c.n_q_heads, c.n_kv_heads, D, c.rms_eps, 1);                      // :444-472
            float* kc = l.kc.data() + (size_t)b * m->cap * m->kvdim;
            float* vc = l.vc.data() + (size_t)b * m->cap * m->kvdim;
            orc_kv_ring_append(kc, vc, qkv.data() + m->qdim, qkv.data() + m->qdim + m->kvdim, m->kvdim,
                               &l.start[b], &l.len[b], m->cap);                               // :475-488
            orc_gqa_attention(attn.data(), qkv.data(), kc, vc, c.n_q_heads, c.n_kv_heads, D, D, l.start[b],
                              l.len[b], m->cap);                                              // :490-492
            project(o.data(), attn.data(), l.o16.data(), H, m->qdim);                         // o_proj
            for (int i = 0; i < H; i++) x[i] = x[i] + o[i];                                   // :516
            orc_rmsnorm(xn.data(), x.data(), l.w_post.data(), H, c.rms_eps);                 // :518
            project(gu.data(), xn.data(), l.gu16.data(), 2 * I, H);                           // fused_ffn: gate|up
            orc_silu_mul(h.data(), gu.data(), gu.data() + I, (size_t)I, 1);
            project(o.data(), h.data(), l.down16.data(), H, I);                               // fused_ffn: down
            for (int i = 0; i < H; i++) x[i] = x[i] + o[i];                                   // :527
        }
        orc_rmsnorm(x.data(), x.data(), m->final_norm.data(), H, c.rms_eps);                 // :530
        project(logits + (size_t)b * c.vocab, x.data(), m->lm16.data(), c.vocab, H);          // LM head
    }
}

extern "C" void orc_qwen3_free(void* m) { delete static_cast<OrcQwen3*>(m); }

// ------------------------------------------------------- KV ring, attention

// models/llm/qwen3.cpp:475-488
extern "C" int orc_kv_ring_append(float* k_cache, float* v_cache, const float* k, const float* v,
                                  int kv_stride, int* start, int* len, int capacity) {
    int slot;
    if (*len < capacity) {                       // :476-479
        slot = *start + *len;
        if (slot >= capacity) slot -= capacity;
        (*len)++;
    } else {                                     // :480-484
        slot = *start;
        (*start)++;
        if (*start >= capacity) *start = 0;
    }
    std::memcpy(k_cache + (size_t)slot * kv_stride, k, (size_t)kv_stride * sizeof(float));  // :487
    std::memcpy(v_cache + (size_t)slot * kv_stride, v, (size_t)kv_stride * sizeof(float));  // :488
    return slot;
}

// core/cpu_ops.cpp:173-240
extern "C" void orc_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                                  int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                                  int cache_start, int cache_len, int cache_capacity) {
    if (cache_len <= 0) {                                           // :177-180
        std::memset(out, 0, (size_t)n_heads * head_dim * sizeof(float));
        return;
    }
    const int groups = n_heads / n_kv_heads;                        // :182
    const float scale = 1.0f / sqrtf((float)head_dim);              // :183
    const size_t kv_step = (size_t)n_kv_heads * head_dim;           // :184
    int first_span = cache_capacity - cache_start;                  // :186-188
    if (first_span > cache_len) first_span = cache_len;
    // heads are independent; the reference runs them in parallel for
    // cache_len >= 128 and n_heads >= 4 (:229-236)
#pragma omp parallel for schedule(static) if (cache_len >= 128 && n_heads >= 4)
    for (int h = 0; h < n_heads; h++) {
        std::vector<float> scores(cache_len);
        const int kv_h = h / groups;
        const float* qh = q + (size_t)h * q_head_stride;
        float* oh = out + (size_t)h * head_dim;
        const size_t off = (size_t)kv_h * head_dim;
        auto row = [&](int t) {                                     // ring order :199-209
            const size_t slot = t < first_span ? (size_t)(cache_start + t) : (size_t)(t - first_span);
            return slot * kv_step + off;
        };
        for (int t = 0; t < cache_len; t++) {
            const float* kh = k_cache + row(t);
            double dot = 0.0;
            for (int d = 0; d < head_dim; d++) dot += (double)qh[d] * (double)kh[d];
            scores[t] = (float)dot * scale;
        }
        orc_softmax(scores.data(), cache_len);                      // :211
        for (int d = 0; d < head_dim; d++) oh[d] = 0.0f;            // :213
        for (int t = 0; t < cache_len; t++) {                       // cblas_saxpy :214-223
            const float* vh = v_cache + row(t);
            const float p = scores[t];
            for (int d = 0; d < head_dim; d++) oh[d] = oh[d] + p * vh[d];
        }
    }
}

// ---------------------------------------------------------------- sampling
// core/sampling.cpp:58-65 (after r is drawn): sequential fp32 cumulative sum.
extern "C" int orc_cdf_walk(const float* p, int V, float r) {
    float cum = 0.0f;
    for (int i = 0; i < V; i++) {
        cum = cum + p[i];
        if (cum >= r) return i;
    }
    return V - 1;
}

// core/sampling.cpp:10-66
extern "C" int orc_sample_token(const float* logits, int V, float temperature, float rep_penalty,
                                int ctx, float freq_penalty, const int32_t* recent, int n_recent,
                                float r, float* probs_out) {
    std::vector<float> adj(logits, logits + V);                    // :13-14
    if (n_recent > 0) {
        int start = std::max(0, n_recent - ctx);                   // :17
        std::map<int, int> freq;                                   // :20-26
        for (int j = start; j < n_recent; j++) {
            int tok = recent[j];
            if (tok >= 0 && tok < V) freq[tok]++;
        }
        for (auto& kv : freq) {                                    // :29-42
            int tok = kv.first, count = kv.second;
            if (rep_penalty > 1.0f) {
                if (adj[(size_t)tok] > 0.0f) adj[(size_t)tok] = adj[(size_t)tok] / rep_penalty;
                else adj[(size_t)tok] = adj[(size_t)tok] * rep_penalty;
            }
            // `adjusted[tok] -= frequency_penalty * count` -- one expression,
            // which clang's default -ffp-contract=on fuses into a single
            // multiply-subtract on the reference's arm64 target.
            if (freq_penalty > 0.0f)
                adj[(size_t)tok] = fmaf(-freq_penalty, (float)count, adj[(size_t)tok]);
        }
    }
    if (temperature <= 0.0f) {                                     // :45-52
        int mi = 0;
        for (int i = 1; i < V; i++)
            if (adj[(size_t)i] > adj[(size_t)mi]) mi = i;
        return mi;
    }
    float inv_t = 1.0f / temperature;                              // :54-55
    for (int i = 0; i < V; i++) adj[(size_t)i] = adj[(size_t)i] * inv_t;
    orc_softmax(adj.data(), V);                                    // :56
    if (probs_out) std::memcpy(probs_out, adj.data(), (size_t)V * sizeof(float));
    return orc_cdf_walk(adj.data(), V, r);                         // :58-65
}

// ---------------------------------------------------------------- layer chain
extern "C" void orc_layer_chain(long T, int H, int nq, int nk, int D, int I, float* x, float* xn,
                                const float* attn_out, const float* mlp_out, float* q, float* k,
                                const float* g, const float* u, float* h, const float* w_in,
                                const float* w_post, const float* wq, const float* wk,
                                const int32_t* pos, const float* cos_tab, const float* sin_tab,
                                int tab_len, float theta, float eps, int nthreads) {
    int nt = nthreads_or_default(nthreads);
    int half = D / 2;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long t = 0; t < T; t++) {
        float* xt = x + (size_t)t * H;
        float* xnt = xn + (size_t)t * H;
        orc_rmsnorm(xnt, xt, w_in, H, eps);                                       // (1)
        float* qt = q + (size_t)t * nq * D;
        float* kt = k + (size_t)t * nk * D;
        for (int hh = 0; hh < nq; hh++) orc_rmsnorm(qt + (size_t)hh * D, qt + (size_t)hh * D, wq, D, eps);
        for (int hh = 0; hh < nk; hh++) orc_rmsnorm(kt + (size_t)hh * D, kt + (size_t)hh * D, wk, D, eps);
        int p = pos[t];
        const float* cr = nullptr;
        const float* sr = nullptr;
        if (p >= 0 && p < tab_len) { cr = cos_tab + (size_t)p * half; sr = sin_tab + (size_t)p * half; }
        orc_rope_qwen3(qt, kt, nq, nk, D, p, theta, cr, sr);                      // (2)
        const float* at = attn_out + (size_t)t * H;
        for (int i = 0; i < H; i++) xt[i] = xt[i] + at[i];                        // (3)
        orc_rmsnorm(xnt, xt, w_post, H, eps);
        const float* gt = g + (size_t)t * I;
        const float* ut = u + (size_t)t * I;
        float* ht = h + (size_t)t * I;
        for (int i = 0; i < I; i++) {                                             // (4)
            float e = expf(-gt[i]);
            e = e + 1.0f;
            ht[i] = (gt[i] / e) * ut[i];
        }
        const float* mt = mlp_out + (size_t)t * H;
        for (int i = 0; i < H; i++) xt[i] = xt[i] + mt[i];                        // (5)
    }
}
