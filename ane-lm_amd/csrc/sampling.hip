// Softmax and batched token sampling for gfx950 (core/cpu_ops.cpp:83-99,
// core/sampling.cpp:10-66).
//
// Floating-point contraction is OFF in this file: every product and sum is
// rounded as written, because the probabilities must be bit-identical to
// the sequential reference formula for the sampled ids to match.
//
// Pipeline per call (rows x vocab; chunks of kCH = 4096 logits, sub-tiles of
// kSub = 256):
//   stage1  grid (chunks, rows): penalties + 1/T, per-chunk max (or argmax)
//   stage2  grid (chunks, rows): e = exp(x - rowmax) into the probability
//           buffer, exact fixed-point chunk sums
//   stage3  grid (chunks, rows): p = e * (1/sum) in place, and for every
//           sub-tile the exact running-sum map under the binade its start is
//           predicted to lie in (see "categorical draw")
//   walk    grid (rows), one wave each: the sequential fp32 CDF walk, passing
//           up to 64 sub-tiles per step where the predictions hold and
//           walking the others exactly, with no barriers
// Stages 1 and 2 recompute the adjusted logit from the input (a few flops)
// instead of storing it; stage 3 reads the exponentials stage 2 stored.
#pragma clang fp contract(off)

#include <climits>
#include <cmath>

#include "anelm_common.hpp"

namespace anelm {

constexpr int kCH = 4096;   // logits per chunk (stage workgroup)
constexpr int kSub = 256;   // logits per walk sub-tile: one wave's part of a k-slice of a chunk

struct SampleArgs {
    const float* logits;
    long ld_logits;
    float* probs;
    long ld_probs;
    int32_t* ids;
    long rows;
    long vocab;
    const int32_t* hist;
    long hist_ld;
    const int32_t* hist_len;
    float rep;
    float freq;
    int ctx;
    int use_penalty;
    int apply_temp;
    float inv_t;
    const float* r;
    uint64_t* ws_sum;     // [rows, nchunk] exact fixed-point sums of exp
    float* ws_max;        // [rows, nchunk] chunk maxima
    int32_t* ws_arg;      // [rows, nchunk] chunk argmax (T <= 0)
    int32_t* ws_flag;     // [rows, nchunk] NaN flags
    uint32_t* ws_map0;    // [rows, nsub] sub-tile map, even start
    uint32_t* ws_map1;    // [rows, nsub] sub-tile map, odd start
    int32_t* ws_cls;      // [rows, nsub] predicted binade class (-1: none)
    int nchunk;
    int nsub;
    int shift;
    int vec_probs;        // probs rows are 16-byte aligned
};

// ---- exp with a fixed IEEE operation sequence ----------------------------
// Cody & Waite two-constant reduction (Software Manual for the Elementary
// Functions, 1980), degree-7 Taylor polynomial by Horner with fused
// multiply-adds, exact power-of-two scaling (two multiplies when the result
// is subnormal so it is rounded once).  Every operation is a correctly
// rounded IEEE operation, so the value is reproducible bit for bit on any
// IEEE machine; it is within 1 ulp of exp.
__device__ __forceinline__ float pow2i(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }

__device__ __forceinline__ float sampler_expf(float x) {
    if (x != x) return x;
    if (x < -104.0f) return 0.0f;
    if (x > 89.0f) return INFINITY;
    const float kf = rintf(x * 0x1.715476p+0f);
    const int k = (int)kf;
    float r = fmaf(-kf, 0x1.63p-1f, x);
    r = fmaf(-kf, -0x1.bd0106p-13f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    if (k < -126) return (p * pow2i(k + 64)) * pow2i(-64);
    if (k > 127) return (p * pow2i(k - 1)) * 2.0f;
    return p * pow2i(k);
}

// ---- history counts --------------------------------------------------------
// cnt[i - c0] = occurrences of id i in the row's window (the last ctx entries,
// sampling.cpp:17) for i in [c0, c0 + n), ids outside [0, vocab) ignored
// (sampling.cpp:23).
__device__ void build_counts(uint32_t* cnt, int n, const SampleArgs& a, long row, long c0) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) cnt[i] = 0u;
    __syncthreads();
    if (a.use_penalty) {
        long hl = a.hist_len ? (long)a.hist_len[row] : a.hist_ld;
        if (hl > a.hist_ld) hl = a.hist_ld;
        long start = hl - a.ctx;
        if (start < 0) start = 0;
        const int32_t* h = a.hist + row * a.hist_ld;
        for (long j = start + threadIdx.x; j < hl; j += blockDim.x) {
            const int id = h[j];
            if (id >= 0 && id < a.vocab && id >= c0 && id < c0 + n) atomicAdd(&cnt[id - c0], 1u);
        }
    }
    __syncthreads();
}

// sampling.cpp:29-42 and :54-55 for one logit whose id occurs n times.
__device__ __forceinline__ float adjust(float l, uint32_t n, const SampleArgs& a) {
    if (n) {
        if (a.rep > 1.0f) l = l > 0.0f ? l / a.rep : l * a.rep;
        // `adjusted[tok] -= frequency_penalty * count`: one fused
        // multiply-subtract, as clang contracts it on the reference's target
        if (a.freq > 0.0f) l = fmaf(-a.freq, (float)n, l);
    }
    if (a.apply_temp) l = l * a.inv_t;
    return l;
}

// The 16 logits of thread tid in chunk c0 (4 float4 slots k*1024 + 4*tid).
__device__ __forceinline__ void load_chunk16(float v[16], const float* row_ptr, long c0, long vocab, bool vec) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const long i = c0 + k * 1024 + 4 * threadIdx.x;
        if (vec && i + 3 < vocab) {
            const float4 f = ld_nt(reinterpret_cast<const float4*>(row_ptr + i));
            v[4 * k] = f.x;
            v[4 * k + 1] = f.y;
            v[4 * k + 2] = f.z;
            v[4 * k + 3] = f.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) v[4 * k + e] = (i + e < vocab) ? row_ptr[i + e] : 0.0f;
        }
    }
}

// max over the row's chunk maxima (any block size, all threads get it)
__device__ float row_max(const SampleArgs& a, long row, float* red) {
    float m = -INFINITY;
    for (int c = threadIdx.x; c < a.nchunk; c += blockDim.x) m = fmaxf(m, a.ws_max[row * a.nchunk + c]);
    m = wave_max(m);
    const int nw = blockDim.x >> 6;
    if (nw == 1) return m;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < nw; w++) m = fmaxf(m, red[w]);
    return m;
}

// 1 / (row sum) from the chunk sums: exact integer total, one rounding to
// float, exact power-of-two scaling, correctly rounded reciprocal
// (cpu_ops.cpp:95-97).  Any block size; the value does not depend on it.
__device__ float row_inv_sum(const SampleArgs& a, long row, uint64_t* red_s, int* red_f) {
    uint64_t s = 0;
    int f = 0;
    for (int c = threadIdx.x; c < a.nchunk; c += blockDim.x) {
        s += a.ws_sum[row * a.nchunk + c];
        f |= a.ws_flag[row * a.nchunk + c];
    }
    s = wave_sum_u64(s);
    f = __any(f) ? 1 : 0;
    const int nw = blockDim.x >> 6;
    if (nw > 1) {
        __syncthreads();
        if ((threadIdx.x & 63) == 0) {
            red_s[threadIdx.x >> 6] = s;
            red_f[threadIdx.x >> 6] = f;
        }
        __syncthreads();
        s = 0;
        f = 0;
        for (int w = 0; w < nw; w++) {
            s += red_s[w];
            f |= red_f[w];
        }
    }
    const float sum = f ? NAN : ldexpf((float)s, -a.shift);
    return 1.0f / sum;
}

// ---- the categorical draw: exact sequential running sums -----------------
// The reference walks cum = fl(cum + p[i]) in index order and returns the
// first i with cum >= r (sampling.cpp:58-65).  While cum stays inside one
// binade [2^e, 2^(e+1)) (or below 2^-126) every representable value is an
// integer multiple m of the binade's ulp u, and
//     fl(cum + p) = (m + q) * u,   q = round-half-even-on-(m+q)(p / u),
// so adding p is "add q", where q depends on m only through an exact tie
// (p/u = n + 1/2) and then only through the parity of m.  Each element is
// therefore a map parity -> increment, the pair (q if m even, q if m odd);
// these maps compose associatively, so prefix compositions are exact.  An
// element whose sum would leave the binade is marked (saturated) and is
// added with one ordinary fp32 add.
constexpr uint32_t kSat = 1u << 30;

struct Fn {
    uint32_t a0, a1;  // increment when the running multiple is even / odd
};

__device__ __forceinline__ uint32_t sat_add(uint32_t x, uint32_t y) {
    const uint32_t s = x + y;  // x, y <= kSat, no wrap
    return s > kSat ? kSat : s;
}

// f applied to a running multiple of the given parity (arithmetic select: a
// conditional on a struct field can become a variable offset into memory)
__device__ __forceinline__ uint32_t pick(Fn f, uint32_t m) {
    return f.a0 + ((f.a1 - f.a0) & (0u - (m & 1u)));
}

// first g, then f
__device__ __forceinline__ Fn compose(Fn g, Fn f) {
    Fn h;
    h.a0 = sat_add(g.a0, (g.a0 & 1u) ? f.a1 : f.a0);
    h.a1 = sat_add(g.a1, (g.a1 & 1u) ? f.a0 : f.a1);
    return h;
}

// A binade class: 0 = zero/subnormal running sums (spacing 2^-149 below
// 2^-126), else the biased exponent E (spacing 2^(E-150) in [2^(E-127), 2^(E-126))).
struct Binade {
    int cls;
    int sh;        // p / u = p * 2^sh
    uint32_t m0;   // cum / u (only for an actual cum)
    uint32_t mhi;  // first multiple outside the binade
    float U;       // upper end of the binade
};

__device__ __forceinline__ Binade binade_of_class(int cls) {
    Binade b;
    b.cls = cls;
    b.m0 = 0;
    if (cls == 0) {
        b.sh = 149;
        b.mhi = 1u << 23;
        b.U = 0x1p-126f;
    } else {
        b.sh = 150 - cls;
        b.mhi = 1u << 24;
        b.U = cls < 254 ? __uint_as_float((uint32_t)(cls + 1) << 23) : INFINITY;
    }
    return b;
}

__device__ __forceinline__ Binade binade_of(float cum) {
    const uint32_t cb = __float_as_uint(cum);
    Binade b = binade_of_class(cb < 0x00800000u ? 0 : (int)(cb >> 23));
    b.m0 = cb < 0x00800000u ? cb : ((cb & 0x7FFFFFu) | 0x800000u);
    return b;
}

// The map of adding p inside binade b (saturated if the sum may leave it).
// Straight-line code: a branch per element costs more than the select.
__device__ __forceinline__ Fn elem_map(float p, const Binade& b) {
    // exact below 2^24 (p < U); clamped above so the conversion is defined
    // for the sums that leave the binade, whose map is replaced anyway
    const float t = fminf(ldexpf(p, b.sh), 0x1p30f);
    const float fl = floorf(t);
    const float fr = t - fl;  // exact
    const uint32_t qi = (uint32_t)fl;
    const uint32_t q = qi + (fr > 0.5f ? 1u : 0u);
    const uint32_t tie = fr == 0.5f ? 1u : 0u;
    const uint32_t odd = qi & 1u;
    const bool leave = !(p < b.U);  // leaves the binade (or NaN): exact add at walk time
    Fn f;
    f.a0 = leave ? kSat : q + (tie & odd);
    f.a1 = leave ? kSat : q + (tie & (odd ^ 1u));
    return f;
}

// DPP lane moves within a wave; lanes without a source get 0, which is the
// identity map (0, 0).  Controls: row_shr:n = 0x110+n, wave_shr:1 = 0x138,
// row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ Fn dpp_fn(Fn v) {
    Fn r;
    r.a0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v.a0, CTRL, ROWMASK, 0xF, false);
    r.a1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v.a1, CTRL, ROWMASK, 0xF, false);
    return r;
}

// inclusive in-order scan of the maps over the 64 lanes
__device__ __forceinline__ Fn wave_scan(Fn v) {
    v = compose(dpp_fn<0x111, 0xF>(v), v);
    v = compose(dpp_fn<0x112, 0xF>(v), v);
    v = compose(dpp_fn<0x114, 0xF>(v), v);
    v = compose(dpp_fn<0x118, 0xF>(v), v);
    v = compose(dpp_fn<0x142, 0xA>(v), v);
    v = compose(dpp_fn<0x143, 0xC>(v), v);
    return v;
}

// ---- stage 1: penalties, 1/T, chunk max (T > 0) or chunk argmax (T <= 0) ----
template <bool ARGMAX>
__global__ __launch_bounds__(256) void sample_stage1_kernel(SampleArgs a, int vec) {
    __shared__ uint32_t cnt[kCH];
    __shared__ float red_v[4];
    __shared__ int red_i[4];
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    float v[16];
    load_chunk16(v, a.logits + row * a.ld_logits, c0, a.vocab, vec != 0);
    build_counts(cnt, kCH, a, row, c0);
    float best = -INFINITY;
    int besti = INT_MAX;
#pragma unroll
    for (int k = 0; k < 4; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int li = k * 1024 + 4 * threadIdx.x + e;
            const long i = c0 + li;
            if (i < a.vocab) {
                const float x = adjust(v[4 * k + e], cnt[li], a);
                if (ARGMAX) {
                    // first index of the maximum among non-NaN values
                    if (x == x && (x > best || (x == best && (int)i < besti))) {
                        best = x;
                        besti = (int)i;
                    }
                } else {
                    best = fmaxf(best, x);
                }
            }
        }
    }
    if (ARGMAX) {
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const float ov = __shfl_xor(best, d);
            const int oi = __shfl_xor(besti, d);
            if (ov > best || (ov == best && oi < besti)) {
                best = ov;
                besti = oi;
            }
        }
        if ((threadIdx.x & 63) == 0) {
            red_v[threadIdx.x >> 6] = best;
            red_i[threadIdx.x >> 6] = besti;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < 4; w++)
                if (red_v[w] > best || (red_v[w] == best && red_i[w] < besti)) {
                    best = red_v[w];
                    besti = red_i[w];
                }
            a.ws_max[row * a.nchunk + blockIdx.x] = best;
            a.ws_arg[row * a.nchunk + blockIdx.x] = besti;
        }
    } else {
        best = wave_max(best);
        if ((threadIdx.x & 63) == 0) red_v[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0)
            a.ws_max[row * a.nchunk + blockIdx.x] = fmaxf(fmaxf(red_v[0], red_v[1]), fmaxf(red_v[2], red_v[3]));
    }
}

// T <= 0 (sampling.cpp:45-52): sequential `if (adj[i] > adj[max_i]) max_i = i`
// from max_i = 0 -- the first maximum among non-NaN values, except that a
// NaN at index 0 can never be replaced.
__global__ __launch_bounds__(64) void sample_argmax_final_kernel(SampleArgs a) {
    const long row = blockIdx.x;
    float best = -INFINITY;
    int besti = INT_MAX;
    for (int c = threadIdx.x; c < a.nchunk; c += 64) {
        const float ov = a.ws_max[row * a.nchunk + c];
        const int oi = a.ws_arg[row * a.nchunk + c];
        if (ov > best || (ov == best && oi < besti)) {
            best = ov;
            besti = oi;
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const float ov = __shfl_xor(best, d);
        const int oi = __shfl_xor(besti, d);
        if (ov > best || (ov == best && oi < besti)) {
            best = ov;
            besti = oi;
        }
    }
    // adjusted logit of id 0: its count in the window
    uint32_t n0 = 0;
    if (a.use_penalty) {
        long hl = a.hist_len ? (long)a.hist_len[row] : a.hist_ld;
        if (hl > a.hist_ld) hl = a.hist_ld;
        long start = hl - a.ctx;
        if (start < 0) start = 0;
        for (long j = start + threadIdx.x; j < hl; j += 64) n0 += a.hist[row * a.hist_ld + j] == 0;
        for (int d = 32; d >= 1; d >>= 1) n0 += __shfl_xor(n0, d);
    }
    if (threadIdx.x == 0) {
        const float x0 = adjust(a.logits[row * a.ld_logits], n0, a);
        a.ids[row] = (x0 != x0 || besti == INT_MAX) ? 0 : besti;
    }
}

// ---- stage 2: exact fixed-point sum of exp(x - max) per chunk ---------------
// floor(e * 2^shift) summed as integers (associative, so independent of the
// reduction order); any NaN term flags the row.  The values e are stored in
// the probability buffer (in place over the logits for softmax: every
// workgroup reads its own chunk before writing it), where stage 3 scales them
// into probabilities without recomputing them.
__global__ __launch_bounds__(256) void sample_stage2_kernel(SampleArgs a, int vec, int vec_out) {
    __shared__ uint32_t cnt[kCH];
    __shared__ float red[4];
    __shared__ uint64_t red_s[4];
    __shared__ int red_f[4];
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    float v[16];
    load_chunk16(v, a.logits + row * a.ld_logits, c0, a.vocab, vec != 0);
    build_counts(cnt, kCH, a, row, c0);
    const float neg = -row_max(a, row, red);
    const float scale = ldexpf(1.0f, a.shift);
    float* out = a.probs + row * a.ld_probs;
    uint64_t acc = 0;
    int nan = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float ev[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int li = k * 1024 + 4 * threadIdx.x + e;
            ev[e] = 0.0f;
            if (c0 + li < a.vocab) {
                const float x = sampler_expf(adjust(v[4 * k + e], cnt[li], a) + neg);
                ev[e] = x;
                if (x >= 0.0f && x <= 1.0f) acc += (uint64_t)(x * scale);
                else nan = 1;
            }
        }
        const long i = c0 + k * 1024 + 4 * threadIdx.x;
        if (vec_out && i + 3 < a.vocab) {  // cached store: stage 3 reads these back
            *reinterpret_cast<float4*>(out + i) = make_float4(ev[0], ev[1], ev[2], ev[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (i + e < a.vocab) out[i + e] = ev[e];
        }
    }
    acc = wave_sum_u64(acc);
    nan = __any(nan) ? 1 : 0;
    if ((threadIdx.x & 63) == 0) {
        red_s[threadIdx.x >> 6] = acc;
        red_f[threadIdx.x >> 6] = nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        a.ws_sum[row * a.nchunk + blockIdx.x] = red_s[0] + red_s[1] + red_s[2] + red_s[3];
        a.ws_flag[row * a.nchunk + blockIdx.x] = red_f[0] | red_f[1] | red_f[2] | red_f[3];
    }
}

// ---- stage 3: probabilities and sub-tile maps --------------------------------
// Wave w's part of k-slice k is the 256 consecutive logits c0 + k*1024 + w*256 +
// [0, 256): sub-tile 16*chunk + 4k + w.  For each, the wave predicts the binade
// of the running sum at the sub-tile's start from the exact prefix of the
// earlier chunks' sums plus this chunk's earlier sub-tile sums, and stores
// the in-order composition of its elements' maps under that binade.  The walk
// uses a map only if the actual running sum turns out to lie in that binade
// and the map shows no element leaving it; otherwise it walks exactly.
__global__ __launch_bounds__(256) void sample_stage3_kernel(SampleArgs a, int vec_out) {
    __shared__ uint64_t red_s[4];
    __shared__ int red_f[4];
    __shared__ float ksum[4][4];  // [k][wave] fp32 sums of exp (prediction only)
    __shared__ float s_prefix;
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    float v[16];  // exp(adjusted - max), as stage 2 stored them
    load_chunk16(v, a.probs + row * a.ld_probs, c0, a.vocab, vec_out != 0);
    const float inv = row_inv_sum(a, row, red_s, red_f);
    // exact prefix of the earlier chunks' sums (prediction of the running sum)
    if (wid == 0) {
        uint64_t pre = 0;
        for (int c = lane; c < (int)blockIdx.x; c += 64) pre += a.ws_sum[row * a.nchunk + c];
        pre = wave_sum_u64(pre);
        if (lane == 0) s_prefix = ldexpf((float)pre, -a.shift);
    }
    float p[16];
    float* out = a.probs + row * a.ld_probs;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float ks = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float e = v[4 * k + j];  // 0 past the end of the row
            ks += e;
            p[4 * k + j] = e * inv;
        }
        ks = wave_sum(ks);
        if (lane == 0) ksum[k][wid] = ks;
        const long i = c0 + k * 1024 + 4 * threadIdx.x;
        if (vec_out && i + 3 < a.vocab) {  // cached store: the walk reads these back
            *reinterpret_cast<float4*>(out + i) = make_float4(p[4 * k], p[4 * k + 1], p[4 * k + 2], p[4 * k + 3]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (i + j < a.vocab) out[i + j] = p[4 * k + j];
        }
    }
    __syncthreads();
    float run = s_prefix;  // running prediction, the same order of additions in every wave
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float here = run;
        for (int w = 0; w < wid; w++) here = here + ksum[k][w];
        const float cpred = here * inv;
        const uint32_t cb = __float_as_uint(cpred);
        const bool ok = cpred == cpred && cpred < INFINITY;
        const int cls = ok ? (cb < 0x00800000u ? 0 : (int)(cb >> 23)) : -1;
        const Binade b = binade_of_class(ok ? cls : 0);
        Fn acc = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const long i = c0 + k * 1024 + 4 * threadIdx.x + j;
            acc = compose(acc, i < a.vocab ? elem_map(p[4 * k + j], b) : Fn{0u, 0u});
        }
        acc = wave_scan(acc);
        const long st = (long)blockIdx.x * 16 + 4 * k + wid;
        if (lane == 63 && st < a.nsub) {
            a.ws_map0[row * a.nsub + st] = acc.a0;
            a.ws_map1[row * a.nsub + st] = acc.a1;
            a.ws_cls[row * a.nsub + st] = cls;
        }
        run = run + ((ksum[k][0] + ksum[k][1]) + (ksum[k][2] + ksum[k][3]));
    }
}

// ---- the walk ------------------------------------------------------------------
// One wave per row; no barriers after the set-up.  The wave passes as many
// 256-probability sub-tiles at once as their stored maps allow and walks the
// others exactly, lane l owning elements 4l..4l+3 of the sub-tile (lane order
// is index order).  The probabilities are read back from the stage-3 output.
constexpr int kSumCache = 4096;  // sub-tile summaries cached in LDS per row
constexpr uint32_t kNoEv = 0xFFFFFFFFu;

// The row's three sub-tile summary arrays (n words each) from global memory
// to LDS by one wave, 16 loads per array and lane in flight before the first
// store: at V = 151936 (594 sub-tiles) that is one memory round trip.  The
// loads use clamped indices (always in bounds, n >= 1), so none waits on a
// branch; only the LDS stores are guarded.
__device__ __forceinline__ void copy3_to_lds(int32_t* d0, const int32_t* s0, int32_t* d1, const int32_t* s1,
                                             int32_t* d2, const int32_t* s2, int n) {
    constexpr int K = 16;
    const int lane = threadIdx.x;
    for (int b = 0; b < n; b += 64 * K) {
        int32_t t0[K], t1[K], t2[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int j = b + k * 64 + lane;
            const int jj = j < n ? j : n - 1;
            t0[k] = s0[jj];
            t1[k] = s1[jj];
            t2[k] = s2[jj];
        }
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int j = b + k * 64 + lane;
            if (j < n) {
                d0[j] = t0[k];
                d1[j] = t1[k];
                d2[j] = t2[k];
            }
        }
    }
}

struct WalkShared {
    uint32_t sm0[kSumCache], sm1[kSumCache];  // sub-tile maps
    int32_t scls[kSumCache];                   // predicted binade classes
};

// Exact walk of sub-tile st from the running sum with bits cb.  Inside one
// binade the running sums of all 256 elements follow from one in-order wave
// scan of their maps; an element that leaves the binade is added with an
// ordinary fp32 add and the scan restarts after it.  Returns true when the
// draw is decided (result set), else updates cb to the sub-tile's end.
__device__ bool walk_subtile(const SampleArgs& a, long st, const float* prow, float r, uint32_t& cb, long& result) {
    const int lane = threadIdx.x;
    const long V = a.vocab;
    const long base = st * kSub;
    const long i0 = base + 4 * lane;
    float p[4];
    if (i0 + 3 < V && a.vec_probs) {
        const float4 q = *reinterpret_cast<const float4*>(prow + i0);
        p[0] = q.x;
        p[1] = q.y;
        p[2] = q.z;
        p[3] = q.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) p[e] = i0 + e < V ? prow[i0 + e] : 0.0f;
    }
    // offsets inside the sub-tile: first unprocessed element, end of the row
    const int nvalid = V - base < kSub ? (int)(V - base) : kSub;
    int s = 0;
    while (true) {
        const Binade b = binade_of(__uint_as_float(cb));
        Fn f[4];
        Fn acc = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int o = 4 * lane + e;
            const Fn m = elem_map(p[e], b);
            const bool in = o >= s && o < nvalid;
            f[e].a0 = in ? m.a0 : 0u;
            f[e].a1 = in ? m.a1 : 0u;
            acc = compose(acc, f[e]);
        }
        const Fn incl = wave_scan(acc);
        const uint32_t tot0 = (uint32_t)__builtin_amdgcn_readlane((int)incl.a0, 63);
        const uint32_t tot1 = (uint32_t)__builtin_amdgcn_readlane((int)incl.a1, 63);
        const Fn x = dpp_fn<0x138, 0xF>(incl);  // the lanes before this one
        uint32_t mm = b.m0 + ((b.m0 & 1u) ? x.a1 : x.a0);
        uint32_t ev = kNoEv, evm = 0;
        float evp = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int o = 4 * lane + e;
            const bool act = ev == kNoEv && o >= s && o < nvalid;
            const uint32_t inc = pick(f[e], mm);
            const bool leave = mm >= b.mhi || inc >= b.mhi - mm;  // leaves the binade
            const uint32_t mn = mm + inc;                          // no wrap: mm < 2^24, inc <= 2^30
            const bool hit = !leave && ldexpf((float)mn, -b.sh) >= r;
            evm = act && leave ? mm : evm;
            evp = act && leave ? p[e] : evp;
            ev = act && leave ? (((uint32_t)o << 1) | 1u) : (act && hit ? (uint32_t)o << 1 : ev);
            mm = act && !leave ? mn : mm;
        }
        const unsigned long long bal = __ballot(ev != kNoEv);
        if (bal == 0) {
            const uint32_t mend = b.m0 + ((b.m0 & 1u) ? tot1 : tot0);
            cb = __float_as_uint(ldexpf((float)mend, -b.sh));
            return false;
        }
        const int first = __ffsll((long long)bal) - 1;
        const uint32_t e0 = (uint32_t)__builtin_amdgcn_readlane((int)ev, first);
        const long ei = base + (long)(e0 >> 1);
        if ((e0 & 1u) == 0) {
            result = ei;
            return true;
        }
        // the reference's fp32 add for the element that leaves the binade
        const float c = ldexpf((float)(uint32_t)__builtin_amdgcn_readlane((int)evm, first), -b.sh) +
                        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(evp), first));
        if (c >= r) {
            result = ei;
            return true;
        }
        if (c != c) {  // NaN probability: no later cum can reach r
            result = V - 1;
            return true;
        }
        cb = __float_as_uint(c);
        s = (int)(e0 >> 1) + 1;
    }
}

// one wave per row and per CU: all of the register file is available to it
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void sample_walk_kernel(SampleArgs a) {
    __shared__ WalkShared sh;
    const int lane = threadIdx.x;
    const long row = blockIdx.x;
    const float r = a.r[row];
    const long V = a.vocab;
    const float* prow = a.probs + row * a.ld_probs;
    const int ncache = a.nsub < kSumCache ? a.nsub : kSumCache;
    copy3_to_lds(reinterpret_cast<int32_t*>(sh.sm0), reinterpret_cast<const int32_t*>(a.ws_map0 + row * a.nsub),
                 reinterpret_cast<int32_t*>(sh.sm1), reinterpret_cast<const int32_t*>(a.ws_map1 + row * a.nsub),
                 sh.scls, a.ws_cls + row * a.nsub, ncache);
    __syncthreads();
    // "cum < r" on bit patterns: cum >= 0, so cum < r <=> bits(cum) < bits(r)
    // for r > 0; for r <= 0 or NaN no sub-tile is passed without a walk
    const uint32_t rb = r > 0.0f ? __float_as_uint(r) : 0u;
    uint32_t cb = 0u;  // bits of the running sum
    long result = V - 1;
    long st = 0;
    while (st < a.nsub) {
        // Pass as many sub-tiles as possible at once: lane j holds sub-tile
        // st + j; the in-order scan of their maps gives each one's end value
        // if every sub-tile before it applies.  The first that does not apply
        // (wrong binade, an element leaving the binade, or end >= r) stops.
        const long idx = st + lane;
        const int ccls = cb < 0x00800000u ? 0 : (int)(cb >> 23);
        const uint32_t m0 = ccls ? ((cb & 0x7FFFFFu) | 0x800000u) : cb;
        const uint32_t mhi = ccls ? (1u << 24) : (1u << 23);
        Fn f = {kSat, kSat};
        if (idx < a.nsub) {
            const int pc = idx < kSumCache ? sh.scls[idx] : a.ws_cls[row * a.nsub + idx];
            if (pc == ccls) {
                f.a0 = idx < kSumCache ? sh.sm0[idx] : a.ws_map0[row * a.nsub + idx];
                f.a1 = idx < kSumCache ? sh.sm1[idx] : a.ws_map1[row * a.nsub + idx];
            }
        }
        const Fn pre = wave_scan(f);
        const uint32_t inc = (m0 & 1u) ? pre.a1 : pre.a0;
        const uint32_t me = m0 + inc;  // inc <= kSat, no wrap
        const uint32_t ce = ccls ? (((uint32_t)ccls << 23) | (me & 0x7FFFFFu)) : me;
        const bool stop = !(inc < mhi - m0) || !(ce < rb);
        const unsigned long long bal = __ballot(stop);
        const int npass = bal ? __ffsll((long long)bal) - 1 : 64;
        if (npass > 0) {
            cb = (uint32_t)__builtin_amdgcn_readlane((int)ce, npass - 1);
            st += npass;
        }
        if (npass < 64 && st < a.nsub) {
            if (walk_subtile(a, st, prow, r, cb, result)) break;
            st += 1;
        }
    }
    if (lane == 0) a.ids[row] = (int32_t)result;
}

static int ceil_log2(long n) {
    int c = 0;
    while ((1L << c) < n) c++;
    return c;
}

struct WsLayout {
    size_t off_sum, off_max, off_arg, off_flag, off_m0, off_m1, off_cls, total;
};

static size_t al16(size_t x) { return (x + 15) & ~(size_t)15; }

static WsLayout ws_layout(long rows, long vocab) {
    const size_t nch = (size_t)((vocab + kCH - 1) / kCH);
    const size_t nsub = (size_t)((vocab + kSub - 1) / kSub);
    const size_t n = (size_t)rows * nch, ns = (size_t)rows * nsub;
    WsLayout l;
    l.off_sum = 0;
    l.off_max = l.off_sum + al16(n * sizeof(uint64_t));
    l.off_arg = l.off_max + al16(n * sizeof(float));
    l.off_flag = l.off_arg + al16(n * sizeof(int32_t));
    l.off_m0 = l.off_flag + al16(n * sizeof(int32_t));
    l.off_m1 = l.off_m0 + al16(ns * sizeof(uint32_t));
    l.off_cls = l.off_m1 + al16(ns * sizeof(uint32_t));
    l.total = l.off_cls + al16(ns * sizeof(int32_t));
    return l;
}

static int bind_workspace(SampleArgs& a, void* ws, size_t ws_bytes, long rows, long vocab, const char* who) {
    const WsLayout l = ws_layout(rows, vocab);
    if (!ws || ws_bytes < l.total)
        return fail(ANELM_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who, l.total,
                    ws ? ws_bytes : (size_t)0);
    if (!aligned16(ws)) return fail(ANELM_ERR_WORKSPACE, "%s: workspace must be 16-byte aligned", who);
    char* b = static_cast<char*>(ws);
    a.ws_sum = reinterpret_cast<uint64_t*>(b + l.off_sum);
    a.ws_max = reinterpret_cast<float*>(b + l.off_max);
    a.ws_arg = reinterpret_cast<int32_t*>(b + l.off_arg);
    a.ws_flag = reinterpret_cast<int32_t*>(b + l.off_flag);
    a.ws_map0 = reinterpret_cast<uint32_t*>(b + l.off_m0);
    a.ws_map1 = reinterpret_cast<uint32_t*>(b + l.off_m1);
    a.ws_cls = reinterpret_cast<int32_t*>(b + l.off_cls);
    a.nchunk = (int)((vocab + kCH - 1) / kCH);
    a.nsub = (int)((vocab + kSub - 1) / kSub);
    a.shift = 63 - ceil_log2(vocab);
    return ANELM_OK;
}

}  // namespace anelm

using namespace anelm;

extern "C" size_t anelm_softmax_workspace_size(long rows, long n) {
    if (rows <= 0 || n <= 0) return 0;
    return ws_layout(rows, n).total;
}

extern "C" size_t anelm_sample_workspace_size(long rows, long vocab) {
    if (rows <= 0 || vocab <= 0) return 0;
    return ws_layout(rows, vocab).total;
}

extern "C" int anelm_softmax(float* x, long rows, long n, long ld, void* workspace, size_t workspace_bytes,
                             void* stream) {
    if (!x) return fail(ANELM_ERR_INVALID, "anelm_softmax: null pointer");
    if (rows <= 0 || rows > 65535 || n <= 0 || n > (1L << 30)) return fail(ANELM_ERR_INVALID, "anelm_softmax: rows=%ld n=%ld", rows, n);
    if (ld < n) return fail(ANELM_ERR_INVALID, "anelm_softmax: ld < n");
    SampleArgs a = {};
    int rc = bind_workspace(a, workspace, workspace_bytes, rows, n, "anelm_softmax");
    if (rc) return rc;
    a.logits = x;
    a.ld_logits = ld;
    a.probs = x;
    a.ld_probs = ld;
    a.rows = rows;
    a.vocab = n;
    a.use_penalty = 0;
    a.apply_temp = 0;
    clear_error();
    hipStream_t st = as_stream(stream);
    const int vec = (ld % 4 == 0) && aligned16(x);
    const dim3 grd((unsigned)a.nchunk, (unsigned)rows);
    sample_stage1_kernel<false><<<grd, 256, 0, st>>>(a, vec);
    sample_stage2_kernel<<<grd, 256, 0, st>>>(a, vec, vec);
    sample_stage3_kernel<<<grd, 256, 0, st>>>(a, vec);
    return launch_status("softmax");
}

extern "C" int anelm_sample(int32_t* ids, float* probs, long ld_probs, const float* logits, long ld_logits,
                            long rows, long vocab, const int32_t* hist, long hist_ld, const int32_t* hist_len,
                            const anelm_sampling_params* params, const float* r, void* workspace,
                            size_t workspace_bytes, void* stream) {
    if (!ids || !logits || !params) return fail(ANELM_ERR_INVALID, "anelm_sample: null pointer");
    if (rows <= 0 || rows > 65535 || vocab <= 0 || vocab > (1L << 30))
        return fail(ANELM_ERR_INVALID, "anelm_sample: rows=%ld vocab=%ld", rows, vocab);
    if (ld_logits < vocab) return fail(ANELM_ERR_INVALID, "anelm_sample: ld_logits < vocab");
    if (probs && ld_probs < vocab) return fail(ANELM_ERR_INVALID, "anelm_sample: ld_probs < vocab");
    if (hist_ld < 0 || (hist_ld > 0 && !hist)) return fail(ANELM_ERR_INVALID, "anelm_sample: history");
    const bool sampling = params->temperature > 0.0f;
    if (sampling && !r) return fail(ANELM_ERR_INVALID, "anelm_sample: r is required when temperature > 0");
    if (sampling && !probs) return fail(ANELM_ERR_INVALID, "anelm_sample: probs is required when temperature > 0");
    SampleArgs a = {};
    int rc = bind_workspace(a, workspace, workspace_bytes, rows, vocab, "anelm_sample");
    if (rc) return rc;
    a.logits = logits;
    a.ld_logits = ld_logits;
    a.probs = probs;
    a.ld_probs = ld_probs;
    a.ids = ids;
    a.rows = rows;
    a.vocab = vocab;
    a.hist = hist;
    a.hist_ld = hist_ld;
    a.hist_len = hist_len;
    a.rep = params->repetition_penalty;
    a.freq = params->frequency_penalty;
    a.ctx = params->repetition_context_size;
    a.use_penalty = hist_ld > 0 ? 1 : 0;
    a.apply_temp = sampling ? 1 : 0;
    a.inv_t = sampling ? 1.0f / params->temperature : 1.0f;
    a.r = r;
    clear_error();
    hipStream_t st = as_stream(stream);
    const int vec = (ld_logits % 4 == 0) && aligned16(logits);
    const dim3 grd((unsigned)a.nchunk, (unsigned)rows);
    if (!sampling) {
        sample_stage1_kernel<true><<<grd, 256, 0, st>>>(a, vec);
        sample_argmax_final_kernel<<<dim3((unsigned)rows), 64, 0, st>>>(a);
        return launch_status("sample(argmax)");
    }
    const int vec_out = probs && (ld_probs % 4 == 0) && aligned16(probs);
    a.vec_probs = vec_out;
    sample_stage1_kernel<false><<<grd, 256, 0, st>>>(a, vec);
    sample_stage2_kernel<<<grd, 256, 0, st>>>(a, vec, vec_out);
    sample_stage3_kernel<<<grd, 256, 0, st>>>(a, vec_out);
    sample_walk_kernel<<<dim3((unsigned)rows), 64, 0, st>>>(a);
    return launch_status("sample");
}
