// Softmax and batched token sampling for gfx950 (core/cpu_ops.cpp:83-99,
// core/sampling.cpp:10-66).
//
// Floating-point contraction is OFF in this file: every product and sum is
// rounded as written, because the probabilities must be bit-identical to
// the sequential reference formula for the sampled ids to match.
//
// Pipeline per call (rows x vocab, chunks of kCH = 4096 logits):
//   stage1  grid (chunks, rows): penalties + 1/T, per-chunk max (or argmax)
//   stage2  grid (chunks, rows): exp(x - rowmax), exact fixed-point chunk sums
//   stage3  grid (chunks, rows): p = e * (1/sum) written to probs
//   walk    grid (rows): exact sequential-fp32 CDF walk -> ids
// Each stage recomputes the adjusted logit from the input (a few flops)
// instead of storing intermediates.
#pragma clang fp contract(off)

#include <climits>
#include <cmath>

#include "anelm_common.hpp"

namespace anelm {

constexpr int kCH = 4096;  // logits per chunk / per walk tile

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
    uint64_t* ws_sum;
    float* ws_max;
    int32_t* ws_arg;
    int32_t* ws_flag;
    int nchunk;
    int shift;
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
// sampling.cpp:17), ids outside [0, vocab) ignored (sampling.cpp:23).
__device__ void build_counts(uint32_t* cnt, const SampleArgs& a, long row, long c0) {
    for (int i = threadIdx.x; i < kCH; i += blockDim.x) cnt[i] = 0u;
    __syncthreads();
    if (a.use_penalty) {
        long hl = a.hist_len ? (long)a.hist_len[row] : a.hist_ld;
        if (hl > a.hist_ld) hl = a.hist_ld;
        long start = hl - a.ctx;
        if (start < 0) start = 0;
        const int32_t* h = a.hist + row * a.hist_ld;
        for (long j = start + threadIdx.x; j < hl; j += blockDim.x) {
            const int id = h[j];
            if (id >= 0 && id < a.vocab && id >= c0 && id < c0 + kCH) atomicAdd(&cnt[id - c0], 1u);
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
            const float4 f = *reinterpret_cast<const float4*>(row_ptr + i);
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

__device__ __forceinline__ float block_max256(float v, float* red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// max over the row's chunk maxima
__device__ float row_max(const SampleArgs& a, long row, float* red) {
    float m = -INFINITY;
    for (int c = threadIdx.x; c < a.nchunk; c += 256) m = fmaxf(m, a.ws_max[row * a.nchunk + c]);
    return block_max256(m, red);
}

// ---- stage 1: penalties, 1/T, chunk max (T > 0) or chunk argmax (T <= 0) ----
template <bool ARGMAX>
__global__ __launch_bounds__(256) void sample_stage1_kernel(SampleArgs a, int vec) {
    __shared__ uint32_t cnt[kCH];
    __shared__ float red_v[4];
    __shared__ int red_i[4];
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    build_counts(cnt, a, row, c0);
    float v[16];
    load_chunk16(v, a.logits + row * a.ld_logits, c0, a.vocab, vec != 0);
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
            // thread 0's own value is already the wave-0 result
            a.ws_max[row * a.nchunk + blockIdx.x] = best;
            a.ws_arg[row * a.nchunk + blockIdx.x] = besti;
        }
    } else {
        best = block_max256(best, red_v);
        if (threadIdx.x == 0) a.ws_max[row * a.nchunk + blockIdx.x] = best;
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
// reduction order); any NaN term flags the row.
__global__ __launch_bounds__(256) void sample_stage2_kernel(SampleArgs a, int vec) {
    __shared__ uint32_t cnt[kCH];
    __shared__ float red[4];
    __shared__ uint64_t red_s[4];
    __shared__ int red_f[4];
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    build_counts(cnt, a, row, c0);
    const float neg = -row_max(a, row, red);
    float v[16];
    load_chunk16(v, a.logits + row * a.ld_logits, c0, a.vocab, vec != 0);
    const float scale = ldexpf(1.0f, a.shift);
    uint64_t acc = 0;
    int nan = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int li = k * 1024 + 4 * threadIdx.x + e;
            if (c0 + li < a.vocab) {
                const float x = sampler_expf(adjust(v[4 * k + e], cnt[li], a) + neg);
                if (x >= 0.0f && x <= 1.0f) acc += (uint64_t)(x * scale);
                else nan = 1;
            }
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

// 1 / (row sum) from the chunk sums: exact integer total, one rounding to
// float, exact power-of-two scaling, correctly rounded reciprocal
// (cpu_ops.cpp:95-97).
__device__ float row_inv_sum(const SampleArgs& a, long row, uint64_t* red_s, int* red_f) {
    uint64_t s = 0;
    int f = 0;
    for (int c = threadIdx.x; c < a.nchunk; c += blockDim.x) {
        s += a.ws_sum[row * a.nchunk + c];
        f |= a.ws_flag[row * a.nchunk + c];
    }
    s = wave_sum_u64(s);
    f = __any(f) ? 1 : 0;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        red_s[threadIdx.x >> 6] = s;
        red_f[threadIdx.x >> 6] = f;
    }
    __syncthreads();
    uint64_t tot = 0;
    int nan = 0;
    const int nw = blockDim.x >> 6;
    for (int w = 0; w < nw; w++) {
        tot += red_s[w];
        nan |= red_f[w];
    }
    const float sum = nan ? NAN : ldexpf((float)tot, -a.shift);
    return 1.0f / sum;
}

// ---- stage 3: probabilities ---------------------------------------------------
__global__ __launch_bounds__(256) void sample_stage3_kernel(SampleArgs a, int vec, int vec_out) {
    __shared__ uint32_t cnt[kCH];
    __shared__ float red[4];
    __shared__ uint64_t red_s[4];
    __shared__ int red_f[4];
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    build_counts(cnt, a, row, c0);
    const float neg = -row_max(a, row, red);
    const float inv = row_inv_sum(a, row, red_s, red_f);
    float v[16];
    load_chunk16(v, a.logits + row * a.ld_logits, c0, a.vocab, vec != 0);
    float* out = a.probs + row * a.ld_probs;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int li = k * 1024 + 4 * threadIdx.x + e;
            p[e] = sampler_expf(adjust(v[4 * k + e], cnt[li], a) + neg) * inv;
        }
        const long i = c0 + k * 1024 + 4 * threadIdx.x;
        if (vec_out && i + 3 < a.vocab) {
            st_nt(reinterpret_cast<float4*>(out + i), make_float4(p[0], p[1], p[2], p[3]));
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (i + e < a.vocab) out[i + e] = p[e];
        }
    }
}

// ---- the categorical draw ----------------------------------------------------
// The reference walks cum = fl(cum + p[i]) in index order and returns the
// first i with cum >= r (sampling.cpp:58-65).  While cum stays inside one
// binade [2^e, 2^(e+1)) (or below 2^-126) every representable value is an
// integer multiple m of the binade's ulp u, and
//     fl(cum + p) = (m + q) * u,   q = round-half-even-on-(m+q)(p / u),
// so adding p is "add q", where q depends on m only through an exact tie
// (p/u = n + 1/2) and then only through the parity of m.  Each element is
// therefore a map parity -> increment, represented by the pair
// (q if m even, q if m odd); these maps compose associatively, so a block
// scan gives every prefix exactly.  An element whose sum would leave the
// binade is added with one ordinary fp32 add and the scan restarts after it
// in the new binade.  Hits (cum >= r) are detected on the exact prefixes.
constexpr uint32_t kSat = 1u << 30;

struct Fn {
    uint32_t a0, a1;  // increment when the running multiple is even / odd
};

__device__ __forceinline__ uint32_t sat_add(uint32_t x, uint32_t y) {
    const uint32_t s = x + y;  // x, y <= kSat, no wrap
    return s > kSat ? kSat : s;
}

// first g, then f
__device__ __forceinline__ Fn compose(Fn g, Fn f) {
    Fn h;
    h.a0 = sat_add(g.a0, (g.a0 & 1u) ? f.a1 : f.a0);
    h.a1 = sat_add(g.a1, (g.a1 & 1u) ? f.a0 : f.a1);
    return h;
}

constexpr int kWalkThreads = 1024;
constexpr unsigned long long kNoEvent = ~0ull;

__global__ __launch_bounds__(kWalkThreads) void sample_walk_kernel(SampleArgs a) {
    __shared__ uint32_t cnt[kCH];
    __shared__ uint32_t s_w0[kWalkThreads / 64], s_w1[kWalkThreads / 64];
    __shared__ unsigned long long s_event;
    __shared__ float s_cum;
    __shared__ float red[16];
    __shared__ uint64_t red_s[16];
    __shared__ int red_f[16];
    const long row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const float r = a.r[row];
    const long V = a.vocab;
    const float* lrow = a.logits + row * a.ld_logits;

    // row max and 1/sum from the stage-1/2 workspace (same values as stage 3)
    float m = -INFINITY;
    for (int c = tid; c < a.nchunk; c += kWalkThreads) m = fmaxf(m, a.ws_max[row * a.nchunk + c]);
    m = wave_max(m);
    if (lane == 0) red[wid] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < kWalkThreads / 64; w++) m = fmaxf(m, red[w]);
    const float neg = -m;
    const float inv = row_inv_sum(a, row, red_s, red_f);

    float cum = 0.0f;
    long s = 0;  // first unprocessed index
    long result = V - 1;
    bool done = false;
    for (long tb = 0; tb < V && !done; tb += kCH) {
        // this tile's probabilities, recomputed exactly as stage 3 writes them
        build_counts(cnt, a, row, tb);
        float pv[4];
        const long i0 = tb + 4 * tid;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const long i = i0 + e;
            pv[e] = i < V ? sampler_expf(adjust(lrow[i], cnt[4 * tid + e], a) + neg) * inv : 0.0f;
        }
        while (true) {
            if (tid == 0) s_event = kNoEvent;
            // binade of cum
            const uint32_t cb = __float_as_uint(cum);
            int sh;
            uint32_t m0, mhi;
            float U;
            if (cb < 0x00800000u) {  // zero or subnormal: spacing 2^-149 up to 2^-126
                sh = 149;
                m0 = cb;
                mhi = 1u << 23;
                U = 0x1p-126f;
            } else {
                const int E = (int)(cb >> 23);
                sh = 150 - E;
                m0 = (cb & 0x7FFFFFu) | 0x800000u;
                mhi = 1u << 24;
                U = E < 254 ? __uint_as_float((uint32_t)(E + 1) << 23) : INFINITY;
            }
            Fn f[4];
            Fn acc = {0u, 0u};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const long i = i0 + e;
                if (i < s || i >= V) {
                    f[e].a0 = f[e].a1 = 0u;
                } else if (!(pv[e] < U)) {  // leaves the binade (or NaN): exact add later
                    f[e].a0 = f[e].a1 = kSat;
                } else {
                    const float t = ldexpf(pv[e], sh);  // exact: p/u < 2^24
                    const float fl = floorf(t);
                    const float fr = t - fl;            // exact
                    const uint32_t qi = (uint32_t)fl;
                    const uint32_t q = qi + (fr > 0.5f ? 1u : 0u);
                    const bool tie = fr == 0.5f;
                    f[e].a0 = q + ((tie && (qi & 1u)) ? 1u : 0u);
                    f[e].a1 = q + ((tie && !(qi & 1u)) ? 1u : 0u);
                }
                acc = compose(acc, f[e]);
            }
            // inclusive wave scan of the per-thread maps
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                Fn b;
                b.a0 = __shfl_up(acc.a0, d);
                b.a1 = __shfl_up(acc.a1, d);
                if (lane >= d) acc = compose(b, acc);
            }
            Fn ex;
            ex.a0 = __shfl_up(acc.a0, 1);
            ex.a1 = __shfl_up(acc.a1, 1);
            if (lane == 0) ex.a0 = ex.a1 = 0u;
            if (lane == 63) {
                s_w0[wid] = acc.a0;
                s_w1[wid] = acc.a1;
            }
            __syncthreads();
            Fn wp = {0u, 0u};
            for (int w = 0; w < wid; w++) wp = compose(wp, Fn{s_w0[w], s_w1[w]});
            const Fn x = compose(wp, ex);
            // walk this thread's elements from the exact prefix
            uint32_t mm = m0 + ((m0 & 1u) ? x.a1 : x.a0);
            unsigned long long ev = kNoEvent;
            uint32_t ev_m = 0;
            float ev_p = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const long i = i0 + e;
                if (ev == kNoEvent && i >= s && i < V) {
                    const uint32_t inc = (mm & 1u) ? f[e].a1 : f[e].a0;
                    if (mm >= mhi || inc >= mhi - mm) {
                        ev = ((unsigned long long)i << 1) | 1ull;  // leaves the binade
                        ev_m = mm;
                        ev_p = pv[e];
                    } else {
                        mm += inc;
                        if (ldexpf((float)mm, -sh) >= r) ev = (unsigned long long)i << 1;  // hit
                    }
                }
            }
            if (ev != kNoEvent) atomicMin(&s_event, ev);
            __syncthreads();
            const unsigned long long evmin = s_event;
            if (evmin == kNoEvent) {
                Fn tot = {0u, 0u};
                for (int w = 0; w < kWalkThreads / 64; w++) tot = compose(tot, Fn{s_w0[w], s_w1[w]});
                const uint32_t mend = m0 + ((m0 & 1u) ? tot.a1 : tot.a0);
                cum = ldexpf((float)mend, -sh);
                s = tb + kCH;
                __syncthreads();
                break;
            }
            const long ei = (long)(evmin >> 1);
            if ((evmin & 1ull) == 0) {
                result = ei;
                done = true;
                __syncthreads();
                break;
            }
            if (ev == evmin) s_cum = ldexpf((float)ev_m, -sh) + ev_p;  // the reference's fp32 add
            __syncthreads();
            cum = s_cum;
            __syncthreads();
            if (cum >= r) {
                result = ei;
                done = true;
                break;
            }
            if (cum != cum) {  // NaN probability: no later cum can reach r
                result = V - 1;
                done = true;
                break;
            }
            s = ei + 1;
        }
        __syncthreads();  // cnt is rebuilt for the next tile
    }
    if (tid == 0) a.ids[row] = (int32_t)result;
}

static int ceil_log2(long n) {
    int c = 0;
    while ((1L << c) < n) c++;
    return c;
}

struct WsLayout {
    size_t off_sum, off_max, off_arg, off_flag, total;
};

static WsLayout ws_layout(long rows, long vocab) {
    const size_t nch = (size_t)((vocab + kCH - 1) / kCH);
    const size_t n = (size_t)rows * nch;
    WsLayout l;
    l.off_sum = 0;
    l.off_max = l.off_sum + n * sizeof(uint64_t);
    l.off_arg = l.off_max + ((n * sizeof(float) + 15) & ~(size_t)15);
    l.off_flag = l.off_arg + ((n * sizeof(int32_t) + 15) & ~(size_t)15);
    l.total = l.off_flag + ((n * sizeof(int32_t) + 15) & ~(size_t)15);
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
    a.nchunk = (int)((vocab + kCH - 1) / kCH);
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
    sample_stage2_kernel<<<grd, 256, 0, st>>>(a, vec);
    sample_stage3_kernel<<<grd, 256, 0, st>>>(a, vec, vec);
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
    sample_stage1_kernel<false><<<grd, 256, 0, st>>>(a, vec);
    sample_stage2_kernel<<<grd, 256, 0, st>>>(a, vec);
    if (probs) {
        const int vec_out = (ld_probs % 4 == 0) && aligned16(probs);
        sample_stage3_kernel<<<grd, 256, 0, st>>>(a, vec, vec_out);
    }
    sample_walk_kernel<<<dim3((unsigned)rows), kWalkThreads, 0, st>>>(a);
    return launch_status("sample");
}
