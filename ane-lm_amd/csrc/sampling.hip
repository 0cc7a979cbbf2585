// Softmax and batched token sampling for gfx950 (core/cpu_ops.cpp:83-99,
// core/sampling.cpp:10-66).
//
// Floating-point contraction is OFF in this file: every product and sum is
// rounded as written, because the probabilities must be bit-identical to
// the sequential reference formula for the sampled ids to match.
//
// Pipeline per call (rows x vocab; chunks of K slices of 1024 logits, K = 3
// unless the call has too few rows to fill the GPU with such chunks, then
// K = 1; sub-tiles of kSub = 256):
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
// With many sampling rows stages 1-3 run as one launch instead (chunks of
// 4, 8 or 12 slices kept in registers, row barriers between the stages; see
// "stages 1-3 in one launch"): the logits are read once and the
// probabilities written once.
#pragma clang fp contract(off)

#include <climits>
#include <cmath>
#include <mutex>

#include "anelm_common.hpp"

namespace anelm {

constexpr int kSlice = 1024;  // logits per k-slice: 4 per thread of a 256-thread workgroup
constexpr int kSub = 256;     // logits per walk sub-tile: one wave's part of a k-slice of a chunk
constexpr int kFirstSubs = 4; // at most sub-tiles 0..3, chunk 0's first k-slice, walked one add at a time by stage 3
constexpr int kFirstN = kFirstSubs * kSub;

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
    uint32_t* ws_xing;    // [rows, nsub, kXWords] predicted crossing (see predict_crossing)
    int32_t* ws_first;    // [rows, 2] sub-tiles 0..first_subs-1 walked by stage 3: hit index or -1, end bits
    // the one-launch path (stages 1-3 in one kernel) only; null otherwise
    uint64_t* ws_tok;     // [rows, 2, nchunk] done flags of its two row barriers
    uint64_t* ws_rowtok;  // [rows, 2] the call's token, and the token again when a row barrier gave up
    uint64_t* epoch;      // one-launch calls made on this workspace (advanced by the walk)
    int first_subs;       // sub-tiles stage 3 walks one add at a time (1 or kFirstSubs)
    int nchunk;
    int nsub;
    int nsub_ld;          // row stride of the sub-tile arrays: nsub rounded up to 4 (16-byte rows)
    int shift;
    int vec_probs;        // probs rows are 16-byte aligned
    float skip_margin;    // stage 3 makes no maps for sub-tiles predicted to start this far past r
};

// ---- exp with a fixed IEEE operation sequence ----------------------------
// Cody & Waite two-constant reduction (Software Manual for the Elementary
// Functions, 1980), degree-7 Taylor polynomial by Horner with fused
// multiply-adds, power-of-two scaling rounded once.  Every operation is a
// correctly rounded IEEE operation, so the value is reproducible bit for bit
// on any IEEE machine; it is within 1 ulp of exp.
__device__ __forceinline__ float sampler_expf(float x) {
    // Straight-line.  The clamp keeps the body finite (maxnum ignores a NaN)
    // and decides the ends: at -104, k = -150 and p = 0x1.f1e6b6p-1, so the
    // scaling gives exactly +0 (0 for x < -104); at 89, k = 128 and
    // p = 0x1.51c2ccp+0, so it gives +inf (inf for x > 89).  A NaN x is
    // selected at the end.
    const float xc = fminf(fmaxf(x, -104.0f), 89.0f);
    const float kf = rintf(xc * 0x1.715476p+0f);
    const int k = (int)kf;
    float r = fmaf(-kf, 0x1.63p-1f, xc);
    r = fmaf(-kf, -0x1.bd0106p-13f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    // p * 2^k rounded once (v_ldexp_f32 is the IEEE scaleB operation): the
    // same value as (p * 2^(k+64)) * 2^-64 for subnormal results,
    // (p * 2^(k-1)) * 2 above 2^127 and p * 2^k otherwise
    const float y = ldexpf(p, k);
    return x != x ? x : y;
}

// ---- history counts --------------------------------------------------------
// The window is the last ctx entries of the row's history (sampling.cpp:17).
// Without hist_len it is known from the arguments, and this thread's first
// entry is loaded by hist_first, ahead of the chunk's logits: loads complete
// in issue order, so the counts can be built while the logits are in flight.
// With hist_len the window waits for that device value (build_counts).
struct HistFirst {
    long hl, start;  // the window is entries [start, hl)
    int raw;         // entry start + min(threadIdx.x, n - 1), as loaded
    bool valid;      // threadIdx.x < n: raw is this thread's first entry
};

// One unconditional load at a clamped index, with no branch (a load inside a
// branch made the compiler wait for it where the branch ends, before the
// chunk's loads went out); nothing uses its value before the chunk's loads
// are issued.  Without such a window the load reads the first logit and the
// value is never used.
__device__ __forceinline__ HistFirst hist_first(const SampleArgs& a, long row) {
    const bool on = a.use_penalty && !a.hist_len && a.hist_ld > 0;   // uniform
    HistFirst f;
    f.hl = on ? a.hist_ld : 0;
    f.start = on && f.hl - a.ctx > 0 ? f.hl - a.ctx : 0;
    const long n = f.hl - f.start;  // >= 1 when on
    f.valid = on && (long)threadIdx.x < n;
    const int32_t* p = on ? a.hist + row * a.hist_ld + f.start + (f.valid ? (long)threadIdx.x : n - 1)
                          : reinterpret_cast<const int32_t*>(a.logits);
    f.raw = *p;
    return f;
}

__device__ __forceinline__ int first_id(const HistFirst& f) { return f.valid ? f.raw : -1; }

// cnt[i - c0] = occurrences of id i in the window for i in [c0, c0 + n)
// (n a multiple of 8), ids outside [0, vocab) ignored (sampling.cpp:23).
// PK: two 16-bit counts per word (id i - c0 in half (i - c0) & 1 of word
// (i - c0) / 2), half the LDS; for windows of at most 65535 ids, so that no
// count carries into its neighbour.
// id0: the window's first entry for this thread (first_id, -1 for none).
template <bool PK = false>
__device__ __forceinline__ void build_counts(uint32_t* cnt, int n, const SampleArgs& a, long row, long c0, HistFirst f,
                                             int id0) {
    const int32_t* h = a.hist + row * a.hist_ld;
    const int words = PK ? n / 2 : n;
    for (int i = 4 * threadIdx.x; i < words; i += 4 * blockDim.x) *reinterpret_cast<uint4*>(cnt + i) = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    auto count = [&](int id) {
        if (id >= 0 && id < a.vocab && id >= c0 && id < c0 + n) {
            const int o = (int)(id - c0);
            if (PK) atomicAdd(&cnt[o >> 1], 1u << (16 * (o & 1)));
            else atomicAdd(&cnt[o], 1u);
        }
    };
    // The two windows in separate branches: a value that one of them loads
    // late (the device length, then the entries) is never the other's, so the
    // first entry's count waits only for its own early load.
    if (a.use_penalty && a.hist_len) {
        long hl = (long)a.hist_len[row];
        if (hl > a.hist_ld) hl = a.hist_ld;
        const long start = hl - a.ctx < 0 ? 0 : hl - a.ctx;
        for (long j = start + threadIdx.x; j < hl; j += blockDim.x) count(h[j]);
    } else if (a.use_penalty) {
        count(id0);
        for (long j = f.start + threadIdx.x + blockDim.x; j < f.hl; j += blockDim.x) count(h[j]);
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

// The 4K adjusted logits of this thread in place (the element order of
// load_chunk); the counts come in K 16-byte LDS reads before any use.
// PK: the counts two per word (build_counts<true>).
template <int K, bool PK = false>
__device__ __forceinline__ void adjust_k(float v[4 * K], const uint32_t* cnt, const SampleArgs& a) {
    uint4 n[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        if constexpr (PK) {
            const uint2 w = *reinterpret_cast<const uint2*>(cnt + (k * kSlice + 4 * threadIdx.x) / 2);
            n[k] = make_uint4(w.x & 0xFFFFu, w.x >> 16, w.y & 0xFFFFu, w.y >> 16);
        } else {
            n[k] = *reinterpret_cast<const uint4*>(cnt + k * kSlice + 4 * threadIdx.x);
        }
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        // Most 256-logit slices of a wave hold no id of the window (256 ids
        // in 151936): there only 1/T applies, adjust() with n = 0.  The
        // branch is wave-uniform.
        if (__ballot((n[k].x | n[k].y | n[k].z | n[k].w) != 0u) == 0) {
            if (a.apply_temp) {
#pragma unroll
                for (int e = 0; e < 4; e++) v[4 * k + e] = v[4 * k + e] * a.inv_t;
            }
            continue;
        }
        v[4 * k] = adjust(v[4 * k], n[k].x, a);
        v[4 * k + 1] = adjust(v[4 * k + 1], n[k].y, a);
        v[4 * k + 2] = adjust(v[4 * k + 2], n[k].z, a);
        v[4 * k + 3] = adjust(v[4 * k + 3], n[k].w, a);
    }
}

// The 4K logits of thread tid in chunk c0 (K float4 slots k*1024 + 4*tid),
// 0 past the end of the row.  An aligned row whose length is a multiple of 4
// takes K 16-byte loads with no branch: every lane loads a quad at a clamped
// index and out-of-range values are selected away afterwards (a branch per
// lane or per chunk made the compiler wait for earlier loads before issuing
// these).  Other rows take single loads.
// In two parts: load_chunk_issue sends the quad loads, load_chunk_finish
// makes the values (the selects wait for the loads).  Work placed between the
// two (the window counts, the row's chunk maxima or sums) runs while the
// chunk is in flight; the element path is complete after the first part.
// Q (the quad path) is a template parameter, not a run-time branch: with both
// paths in one kernel the compiler joined them before the quad loads and
// waited there for every load issued earlier.
__host__ __device__ inline bool chunk_quads(long vocab, bool vec) { return vec && vocab >= 4 && (vocab & 3) == 0; }

template <int K, bool Q>
__device__ __forceinline__ void load_chunk_issue(float4 (&f)[K], float (&v)[4 * K], const float* row_ptr, long c0, long vocab) {
    if constexpr (Q) {
        const long lastq = vocab - 4;  // the last quad
#pragma unroll
        for (int k = 0; k < K; k++) {
            const long i = c0 + k * kSlice + 4 * threadIdx.x;
            f[k] = ld_nt(reinterpret_cast<const float4*>(row_ptr + (i < lastq ? i : lastq)));
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; k++) {
            const long i = c0 + k * kSlice + 4 * threadIdx.x;
#pragma unroll
            for (int e = 0; e < 4; e++) v[4 * k + e] = (i + e < vocab) ? row_ptr[i + e] : 0.0f;
        }
        // complete here: where a run-time branch picks this path or the
        // quad loads, nothing of it is left pending where the paths join
        __builtin_amdgcn_s_waitcnt(0);
    }
}

template <int K, bool Q>
__device__ __forceinline__ void load_chunk_finish(float (&v)[4 * K], const float4 (&f)[K], long c0, long vocab) {
    if constexpr (Q) {
#pragma unroll
        for (int k = 0; k < K; k++) {
            const long i = c0 + k * kSlice + 4 * threadIdx.x;
            const bool in = i + 3 < vocab;
            v[4 * k] = in ? f[k].x : 0.0f;
            v[4 * k + 1] = in ? f[k].y : 0.0f;
            v[4 * k + 2] = in ? f[k].z : 0.0f;
            v[4 * k + 3] = in ? f[k].w : 0.0f;
        }
    }
}

// The row's chunk maxima and chunk sums are read by every workgroup of the
// next stage.  Each thread loads its share first (the loads do not depend on
// the chunk's own data, so their latency overlaps the chunk loads), and the
// workgroup reduces the shares later.

// this thread's share of the row max: its first chunk maximum (one
// unconditional load at a clamped index, selected only after the chunk's
// loads are issued: a use would wait for it), then any others
__device__ __forceinline__ float max_first(const SampleArgs& a, long row) {
    const int c = (int)threadIdx.x < a.nchunk ? (int)threadIdx.x : a.nchunk - 1;
    return a.ws_max[row * a.nchunk + c];
}
__device__ __forceinline__ float max_rest(const SampleArgs& a, long row, float raw) {
    float m = (int)threadIdx.x < a.nchunk ? raw : -INFINITY;
    for (int c = threadIdx.x + blockDim.x; c < a.nchunk; c += blockDim.x) m = fmaxf(m, a.ws_max[row * a.nchunk + c]);
    return m;
}

// the row max from the shares (any block size, all threads get it)
__device__ float reduce_max(float m, float* red) {
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

// this thread's share of the row sum, of the sum of the chunks before chunk
// `before`, and of the NaN flags
struct SumShare {
    uint64_t all, pre;
    int flag;
};

// its first chunk's values (unconditional loads at a clamped index, used
// only after the chunk's loads are issued), then any others
struct SumRaw {
    uint64_t w;
    int f;
};
__device__ __forceinline__ SumRaw sum_first(const SampleArgs& a, long row) {
    const int c = (int)threadIdx.x < a.nchunk ? (int)threadIdx.x : a.nchunk - 1;
    return SumRaw{a.ws_sum[row * a.nchunk + c], a.ws_flag[row * a.nchunk + c]};
}
__device__ __forceinline__ SumShare sum_rest(const SampleArgs& a, long row, int before, SumRaw raw) {
    const int c0 = threadIdx.x;
    const bool in = c0 < a.nchunk;
    SumShare sh = {in ? raw.w : 0u, in && c0 < before ? raw.w : 0u, in ? raw.f : 0};
    for (int c = threadIdx.x + blockDim.x; c < a.nchunk; c += blockDim.x) {
        const uint64_t w = a.ws_sum[row * a.nchunk + c];
        sh.all += w;
        sh.pre += c < before ? w : 0;
        sh.flag |= a.ws_flag[row * a.nchunk + c];
    }
    return sh;
}

// 1 / (row sum) from the shares: exact integer total, one rounding to float,
// exact power-of-two scaling, correctly rounded reciprocal (cpu_ops.cpp:95-97),
// and the prefix as a float (a prediction only).  Any block size; the values
// do not depend on it.
__device__ __forceinline__ void reduce_sums(SumShare sh, const SampleArgs& a, uint64_t* red_s, uint64_t* red_p, int* red_f,
                            float& inv, float& prefix) {
    uint64_t s = wave_sum_u64(sh.all), pre = wave_sum_u64(sh.pre);
    int f = __any(sh.flag) ? 1 : 0;
    const int nw = blockDim.x >> 6;
    if (nw > 1) {
        __syncthreads();
        if ((threadIdx.x & 63) == 0) {
            red_s[threadIdx.x >> 6] = s;
            red_p[threadIdx.x >> 6] = pre;
            red_f[threadIdx.x >> 6] = f;
        }
        __syncthreads();
        s = 0;
        pre = 0;
        f = 0;
        for (int w = 0; w < nw; w++) {
            s += red_s[w];
            pre += red_p[w];
            f |= red_f[w];
        }
    }
    const float sum = f ? NAN : ldexpf((float)s, -a.shift);
    inv = 1.0f / sum;
    prefix = ldexpf((float)pre, -a.shift);
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

// The same scan when no lane's map depends on the parity (a0 == a1 in every
// lane, i.e. no exact rounding tie): composition is then saturating
// addition, which is associative and commutative on [0, kSat].
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_scan_sat(uint32_t v) {
    v = sat_add(dpp_u32<0x111, 0xF>(v), v);
    v = sat_add(dpp_u32<0x112, 0xF>(v), v);
    v = sat_add(dpp_u32<0x114, 0xF>(v), v);
    v = sat_add(dpp_u32<0x118, 0xF>(v), v);
    v = sat_add(dpp_u32<0x142, 0xA>(v), v);
    v = sat_add(dpp_u32<0x143, 0xC>(v), v);
    return v;
}

// In-order scan of per-lane maps, the cheap way when the wave has no tie.
__device__ __forceinline__ Fn wave_scan_any(Fn v) {
    if (__ballot(v.a0 != v.a1) == 0) {
        const uint32_t t = wave_scan_sat(v.a0);
        return Fn{t, t};
    }
    return wave_scan(v);
}

// A lane's four element maps composed in order, and the wave's inclusive
// scan of those compositions; `tie` says whether any map had a0 != a1.
__device__ __forceinline__ Fn compose4_scan(const Fn f[4]) {
    bool tie = false;
#pragma unroll
    for (int j = 0; j < 4; j++) tie = tie || f[j].a0 != f[j].a1;
    if (__ballot(tie) == 0) {
        const uint32_t t = wave_scan_sat(sat_add(sat_add(f[0].a0, f[1].a0), sat_add(f[2].a0, f[3].a0)));
        return Fn{t, t};
    }
    Fn acc = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; j++) acc = compose(acc, f[j]);
    return wave_scan(acc);
}

// ---- stage 1: penalties, 1/T, chunk max (T > 0) or chunk argmax (T <= 0) ----
template <bool ARGMAX, int K, bool Q>
__global__ __launch_bounds__(256) void sample_stage1_kernel(SampleArgs a) {
    constexpr int kCH = K * kSlice;
    __shared__ __align__(16) uint32_t cnt[kCH];
    __shared__ float red_v[4];
    __shared__ int red_i[4];
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    const HistFirst hf = hist_first(a, row);
    __builtin_amdgcn_sched_barrier(0);  // its load goes out before the chunk's
    float v[4 * K];
    float4 q[K];
    load_chunk_issue<K, Q>(q, v, a.logits + row * a.ld_logits, c0, a.vocab);
    __builtin_amdgcn_sched_barrier(0);
    build_counts(cnt, kCH, a, row, c0, hf, first_id(hf));   // while the chunk is in flight
    load_chunk_finish<K, Q>(v, q, c0, a.vocab);
    adjust_k<K>(v, cnt, a);
    const int nvalid = a.vocab - c0 < kCH ? (int)(a.vocab - c0) : kCH;
    float best = -INFINITY;
    int besti = INT_MAX;
#pragma unroll
    for (int k = 0; k < K; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int li = k * kSlice + 4 * threadIdx.x + e;
            const float x = v[4 * k + e];
            if (ARGMAX) {
                // first index of the maximum among non-NaN values
                const int i = (int)c0 + li;
                if (li < nvalid && x == x && (x > best || (x == best && i < besti))) {
                    best = x;
                    besti = i;
                }
            } else {
                best = li < nvalid ? fmaxf(best, x) : best;
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

// A lane's sum of floor(e * 2^shift) over its exponentials.  When its 4K
// terms (each at most 2^shift) stay below 2^53 the sum is kept in fp64:
// widening, scaling by 2^shift, floor and add are then all exact (4
// instructions a term, against about 10 for a float -> u64 floor and a 64-bit
// add), and a NaN or inf term leaves it non-finite.  Otherwise in u64.
template <bool F64>
struct LaneSum {
    double d = 0.0;
    uint64_t u = 0;
    int nan = 0;
    __device__ __forceinline__ void add(float x, float scale, double scaled) {
        if constexpr (F64) {
            d += floor((double)x * scaled);
        } else {
            const bool ok = x <= 1.0f;  // e >= 0 always; false for NaN and inf
            u += (uint64_t)(ok ? x * scale : 0.0f);
            nan |= ok ? 0 : 1;
        }
    }
    __device__ __forceinline__ void finish(uint64_t& acc, int& bad) const {
        if constexpr (F64) {
            const bool b = !(d <= 0x1p53);
            bad = b ? 1 : 0;
            acc = b ? 0u : (uint64_t)d;
        } else {
            bad = nan;
            acc = u;
        }
    }
};

// The chunk's exponentials e = exp(x - max), stored into the probability
// buffer (cached: stage 3 reads them back), and this lane's sum of them.
template <int K, bool F64>
__device__ __forceinline__ void exp_and_sum(const float (&v)[4 * K], float neg, const SampleArgs& a, long row, long c0,
                                            int nvalid, int vec_out, uint64_t& acc, int& nan) {
    constexpr int kCH = K * kSlice;
    const float scale = ldexpf(1.0f, a.shift);
    const double scaled = ldexp(1.0, a.shift);
    float* out = a.probs + row * a.ld_probs;
    LaneSum<F64> sum;
    if (nvalid == kCH && vec_out) {
        // a whole chunk: no per-element bounds (a guard per element compiled
        // to an exec-mask branch per element)
#pragma unroll
        for (int k = 0; k < K; k++) {
            float ev[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                ev[e] = sampler_expf(v[4 * k + e] + neg);
                sum.add(ev[e], scale, scaled);
            }
            *reinterpret_cast<float4*>(out + c0 + k * kSlice + 4 * threadIdx.x) = make_float4(ev[0], ev[1], ev[2], ev[3]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; k++) {
            float ev[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int li = k * kSlice + 4 * threadIdx.x + e;
                ev[e] = li < nvalid ? sampler_expf(v[4 * k + e] + neg) : 0.0f;
                sum.add(ev[e], scale, scaled);
            }
            const long i = c0 + k * kSlice + 4 * threadIdx.x;
            if (vec_out && i + 3 < a.vocab) {
                *reinterpret_cast<float4*>(out + i) = make_float4(ev[0], ev[1], ev[2], ev[3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (i + e < a.vocab) out[i + e] = ev[e];
            }
        }
    }
    sum.finish(acc, nan);
}

// The same exponentials kept in v (0 past the end of the row) instead of
// stored, and this lane's sum of them.  The exp is computed for every slot
// and the padding selected away (no branch per element).
// FULL: every slot is in the row (nvalid == K * kSlice), no selects.
template <int K, bool F64, bool FULL>
__device__ __forceinline__ void exp_and_sum_keep(float (&v)[4 * K], float neg, const SampleArgs& a, int nvalid,
                                                 uint64_t& acc, int& nan) {
    const float scale = ldexpf(1.0f, a.shift);
    const double scaled = ldexp(1.0, a.shift);
    LaneSum<F64> sum;
#pragma unroll
    for (int k = 0; k < K; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int li = k * kSlice + 4 * threadIdx.x + e;
            const float ev = sampler_expf(v[4 * k + e] + neg);
            v[4 * k + e] = FULL || li < nvalid ? ev : 0.0f;
            sum.add(v[4 * k + e], scale, scaled);
        }
    }
    sum.finish(acc, nan);
}

// ---- stage 2: exact fixed-point sum of exp(x - max) per chunk ---------------
// floor(e * 2^shift) summed as integers (associative, so independent of the
// reduction order); any NaN term flags the row.  The values e are stored in
// the probability buffer (in place over the logits for softmax: every
// workgroup reads its own chunk before writing it), where stage 3 scales them
// into probabilities without recomputing them.
template <int K, bool Q>
__global__ __launch_bounds__(256) void sample_stage2_kernel(SampleArgs a, int vec_out) {
    constexpr int kCH = K * kSlice;
    __shared__ __align__(16) uint32_t cnt[kCH];
    __shared__ float red[4];
    __shared__ uint64_t red_s[4];
    __shared__ int red_f[4];
    const long row = blockIdx.y;
    const long c0 = (long)blockIdx.x * kCH;
    // the row's chunk maxima and this thread's window entry first: loads
    // complete in issue order, so their waits do not wait for the logits
    const float mraw = max_first(a, row);
    const HistFirst hf = hist_first(a, row);
    __builtin_amdgcn_sched_barrier(0);
    float v[4 * K];
    float4 q[K];
    load_chunk_issue<K, Q>(q, v, a.logits + row * a.ld_logits, c0, a.vocab);
    __builtin_amdgcn_sched_barrier(0);
    const float mshare = max_rest(a, row, mraw);
    build_counts(cnt, kCH, a, row, c0, hf, first_id(hf));   // while the chunk is in flight
    load_chunk_finish<K, Q>(v, q, c0, a.vocab);
    adjust_k<K>(v, cnt, a);
    const int nvalid = a.vocab - c0 < kCH ? (int)(a.vocab - c0) : kCH;
    const float neg = -reduce_max(mshare, red);
    constexpr int kLogTerms = K == 1 ? 2 : K == 2 ? 3 : K <= 4 ? 4 : K <= 8 ? 5 : 6;  // ceil(log2(4K)), a lane's terms
    uint64_t acc;
    int nan;
    if (a.shift + kLogTerms <= 53)  // uniform: the lane's sum fits fp64's 53 bits
        exp_and_sum<K, true>(v, neg, a, row, c0, nvalid, vec_out, acc, nan);
    else
        exp_and_sum<K, false>(v, neg, a, row, c0, nvalid, vec_out, acc, nan);
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

// ---- crossings: a sub-tile in which the running sum enters the next binade ----
// Inside such a sub-tile the single-binade map cannot pass the walk.  Stage 3
// predicts where the crossing happens (from its prediction of the running
// sum at the sub-tile's start) and stores what the walk needs to pass the
// sub-tile in O(1) if the prediction holds for the actual running sum:
//   pre  the map of the elements before the crossing element j, under the
//        start binade;
//   pj   the crossing element's probability (added with one fp32 add);
//   sfx  the map of the elements after j, under the binade the sum enters;
//   info j | (that binade's class << 8), or -1 when there is no single
//        predicted crossing (none, or a second one in the same sub-tile).
// The walk checks every assumption against the exact running sum and walks
// the sub-tile exactly when one fails, so a wrong prediction costs time only.
constexpr int kXWords = 6;  // words per sub-tile: pre.a0, pre.a1, sfx.a0, sfx.a1, pj, info

struct Crossing {
    Fn pre, sfx;
    float pj;
    int info;
};

// acc: the inclusive scan of the lanes' maps under binade b (class cls);
// f: this lane's four element maps; p: its four probabilities; nv: valid
// elements in the sub-tile; cb: bits of the predicted running sum at its
// start.  Wave-uniform control flow.
__device__ __forceinline__ Crossing predict_crossing(Fn acc, const Fn f[4], const float p[4], int nv, bool ok,
                                                     uint32_t cb, int cls, const Binade& b) {
    Crossing x = {{0u, 0u}, {0u, 0u}, 0.0f, -1};
    const int lane = threadIdx.x & 63;
    const uint32_t t0 = (uint32_t)__builtin_amdgcn_readlane((int)acc.a0, 63);
    const uint32_t t1 = (uint32_t)__builtin_amdgcn_readlane((int)acc.a1, 63);
    const uint32_t mp = cls == 0 ? cb : ((cb & 0x7FFFFFu) | 0x800000u);  // predicted start multiple
    const uint32_t tinc = (mp & 1u) ? t1 : t0;
    if (!ok || tinc < b.mhi - mp) return x;  // no crossing predicted
    // the first element at which the predicted sum leaves binade b
    const Fn ex = dpp_fn<0x138, 0xF>(acc);  // composition of the lanes before this one
    uint32_t mm = mp + pick(ex, mp);
    Fn run = ex, pre = {0u, 0u};
    int ev = kSub;
    uint32_t mb = 0;
    float pe = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int o = 4 * lane + j;
        const bool act = ev == kSub && o < nv;
        const uint32_t inc = pick(f[j], mm);
        const bool leave = mm >= b.mhi || inc >= b.mhi - mm;
        if (act && leave) {
            ev = o;
            mb = mm;
            pe = p[j];
            pre = run;
        }
        mm = act && !leave ? mm + inc : mm;
        run = compose(run, f[j]);
    }
    const unsigned long long bal = __ballot(ev != kSub);
    if (bal == 0) return x;
    const int L = __ffsll((long long)bal) - 1;
    const int jstar = __builtin_amdgcn_readlane(ev, L);
    x.pre.a0 = (uint32_t)__builtin_amdgcn_readlane((int)pre.a0, L);
    x.pre.a1 = (uint32_t)__builtin_amdgcn_readlane((int)pre.a1, L);
    x.pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), L));
    const uint32_t mbs = (uint32_t)__builtin_amdgcn_readlane((int)mb, L);
    // the predicted sum after the crossing add, and the elements after it
    const float c = ldexpf((float)mbs, -b.sh) + x.pj;
    if (!(c < INFINITY)) return x;  // NaN or overflow: no prediction
    const uint32_t c2 = __float_as_uint(c);
    const int cls2 = c2 < 0x00800000u ? 0 : (int)(c2 >> 23);
    const Binade b2 = binade_of_class(cls2);
    Fn gf[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int o = 4 * lane + j;
        const Fn m = elem_map(p[j], b2);
        const bool in = o > jstar && o < nv;
        gf[j] = Fn{in ? m.a0 : 0u, in ? m.a1 : 0u};
    }
    const Fn g = compose4_scan(gf);
    x.sfx.a0 = (uint32_t)__builtin_amdgcn_readlane((int)g.a0, 63);
    x.sfx.a1 = (uint32_t)__builtin_amdgcn_readlane((int)g.a1, 63);
    const uint32_t m2 = cls2 == 0 ? c2 : ((c2 & 0x7FFFFFu) | 0x800000u);
    const uint32_t sinc = (m2 & 1u) ? x.sfx.a1 : x.sfx.a0;
    if (sinc < b2.mhi - m2) x.info = jstar | (cls2 << 8);  // else a second crossing: walk exactly
    return x;
}

__device__ bool walk_subtile_p(const float p[4], long base, long V, float r, uint32_t& cb, long& result);
__device__ bool walk_first_lds(const float* sp, int nsubs, long V, float r, uint32_t& cb, long& result);

// ---- stage 3: probabilities and sub-tile maps --------------------------------
// Wave w's part of k-slice k is the 256 consecutive logits c0 + k*1024 + w*256 +
// [0, 256): sub-tile 4K*chunk + 4k + w.  For each, the wave predicts the binade
// of the running sum at the sub-tile's start from the exact prefix of the
// earlier chunks' sums plus this chunk's earlier sub-tile sums, and stores
// the in-order composition of its elements' maps under that binade.  The walk
// uses a map only if the actual running sum turns out to lie in that binade
// and the map shows no element leaving it; otherwise it walks exactly.
// Stage 3's work once the chunk's exponentials v (0 past the end of the row),
// 1/sum and the exact prefix of the earlier chunks' sums are known: the
// probabilities, the first sub-tiles' walk (chunk 0) and the sub-tile maps.
// ksum and s_first are the workgroup's LDS.
template <int K>
__device__ __forceinline__ void probs_and_maps(const SampleArgs& a, const float (&v)[4 * K], long row, int chunk,
                                               float inv, float prefix, float rdraw, int vec_out, float (*ksum)[4],
                                               float* s_first) {
    constexpr int kCH = K * kSlice;
    const long c0 = (long)chunk * kCH;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    // p = e * (1/sum), one rounding: made here for the stores and again from
    // the same e where the maps need it, so only the exponentials stay live
    // across the walk and the maps (the same bits, fewer registers)
    float* out = a.probs + row * a.ld_probs;
#pragma unroll
    for (int k = 0; k < K; k++) {
        float ks = 0.f;
        float p[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float e = v[4 * k + j];  // 0 past the end of the row
            ks += e;
            p[j] = e * inv;
        }
        ks = wave_sum(ks);
        if (lane == 0) ksum[k][wid] = ks;
        const long i = c0 + k * kSlice + 4 * threadIdx.x;
        if (vec_out && i + 3 < a.vocab) {  // cached store: the walk reads these back
            *reinterpret_cast<float4*>(out + i) = make_float4(p[0], p[1], p[2], p[3]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (i + j < a.vocab) out[i + j] = p[j];
        }
    }
    // The row's first sub-tiles start from an exact running sum, 0, that is
    // small against single elements: it crosses a binade at about every
    // doubling, often twice in one sub-tile, where the map-based walk needs
    // exact walks with restarts.  Lane 0 of each row's first workgroup
    // (dispatched first) walks the first first_subs sub-tiles (of its first
    // k-slice, which its four waves stage in LDS) here instead, one fp32 add
    // at a time, at raised issue priority, while the rest of the grid runs
    // (and the workgroup's other waves make their maps), off the walk
    // kernel's critical path.  With many rows that is four sub-tiles (their
    // exact walks were most of the slowest rows' extra walk time); with a few
    // rows stage 3 is too short to hide more than one.
    if (chunk == 0 && a.r)
        *reinterpret_cast<float4*>(&s_first[wid * kSub + 4 * lane]) =
            make_float4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    __syncthreads();  // ksum and s_first complete; the other waves need not wait for the walk below
    if (chunk == 0 && wid == 0 && a.r) {
        __builtin_amdgcn_s_setprio(3);
        if (lane == 0) {
            uint32_t cb = 0u;
            long result = -1;
            const bool done = walk_first_lds(s_first, a.first_subs, a.vocab, rdraw, cb, result);
            a.ws_first[2 * row] = done ? (int32_t)result : -1;
            a.ws_first[2 * row + 1] = (int32_t)cb;
        }
        __builtin_amdgcn_s_setprio(0);
    }
    float run = prefix;  // running prediction, the same order of additions in every wave
#pragma unroll
    for (int k = 0; k < K; k++) {
        float here = run;
        for (int w = 0; w < wid; w++) here = here + ksum[k][w];
        const float cpred = here * inv;
        const long st = (long)chunk * (4 * K) + 4 * k + wid;
        // No map where the walk does not arrive: without a draw (softmax), for
        // sub-tiles 0..first_subs-1 (walked exactly above; the walk starts
        // after them), or
        // when the sub-tile is predicted to start more than skip_margin past
        // r (the sequential sum is within V * 2^-25 of the exact prefix, so
        // the draw has ended before it).  A wrong prediction costs the walk an
        // exact walk of the sub-tile (class -1, no crossing), never a result.
        if (!a.r || st < a.first_subs || cpred >= rdraw + a.skip_margin) {  // wave-uniform
            if (a.r && lane == 63 && st < a.nsub) {
                a.ws_cls[row * a.nsub_ld + st] = -1;
                a.ws_xing[(row * a.nsub_ld + st) * kXWords + 5] = 0xFFFFFFFFu;
            }
            run = run + ((ksum[k][0] + ksum[k][1]) + (ksum[k][2] + ksum[k][3]));
            continue;
        }
        const uint32_t cb = __float_as_uint(cpred);
        const bool ok = cpred == cpred && cpred < INFINITY;
        const int cls = ok ? (cb < 0x00800000u ? 0 : (int)(cb >> 23)) : -1;
        const Binade b = binade_of_class(ok ? cls : 0);
        const int nv = a.vocab - (c0 + k * kSlice + 256 * wid) < kSub ? (int)(a.vocab - (c0 + k * kSlice + 256 * wid))
                                                                       : kSub;  // valid elements of the sub-tile
        const float p[4] = {v[4 * k] * inv, v[4 * k + 1] * inv, v[4 * k + 2] * inv, v[4 * k + 3] * inv};
        Fn f[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const Fn m = elem_map(p[j], b);
            const bool in = 4 * lane + j < nv;
            f[j].a0 = in ? m.a0 : 0u;
            f[j].a1 = in ? m.a1 : 0u;
        }
        const Fn acc = compose4_scan(f);
        const Crossing x = predict_crossing(acc, f, p, nv, ok, cb, cls, b);
        if (lane == 63 && st < a.nsub) {
            a.ws_map0[row * a.nsub_ld + st] = acc.a0;
            a.ws_map1[row * a.nsub_ld + st] = acc.a1;
            a.ws_cls[row * a.nsub_ld + st] = cls;
            uint32_t* xw = a.ws_xing + (row * a.nsub_ld + st) * kXWords;
            xw[0] = x.pre.a0;
            xw[1] = x.pre.a1;
            xw[2] = x.sfx.a0;
            xw[3] = x.sfx.a1;
            xw[4] = __float_as_uint(x.pj);
            xw[5] = (uint32_t)x.info;
        }
        run = run + ((ksum[k][0] + ksum[k][1]) + (ksum[k][2] + ksum[k][3]));
    }
}

template <int K, bool Q>
__global__ __launch_bounds__(256) void sample_stage3_kernel(SampleArgs a, int vec_out) {
    constexpr int kCH = K * kSlice;
    __shared__ uint64_t red_s[4], red_p[4];
    __shared__ int red_f[4];
    __shared__ float ksum[K][4];  // [k][wave] fp32 sums of exp (prediction only)
    __shared__ __align__(16) float s_first[kFirstN];  // the first k-slice's probabilities for the one-lane walk
    // Workgroups in dispatch order take chunk 0 of every row first: those
    // also walk sub-tiles 0..3 (below), the longest job, so it starts early.
    const long lin = (long)blockIdx.y * gridDim.x + blockIdx.x;
    const long row = lin % a.rows;
    const int chunk = (int)(lin / a.rows);
    const long c0 = (long)chunk * kCH;
    // the draw is loaded with the exponentials (the first sub-tile's walk
    // below compares against it), not behind them
    const float rdraw = a.r ? a.r[row] : 0.0f;
    // and the chunk sums, so that the reduction below does not wait for them
    const SumRaw sraw = sum_first(a, row);
    __builtin_amdgcn_sched_barrier(0);
    float v[4 * K];  // exp(adjusted - max), as stage 2 stored them
    float4 q[K];
    load_chunk_issue<K, Q>(q, v, a.probs + row * a.ld_probs, c0, a.vocab);
    __builtin_amdgcn_sched_barrier(0);
    const SumShare share = sum_rest(a, row, chunk, sraw);
    // 1/sum, and the exact prefix of the earlier chunks' sums (the prediction
    // of the running sum at this chunk's start), while the chunk is in flight
    float inv, prefix;
    reduce_sums(share, a, red_s, red_p, red_f, inv, prefix);
    load_chunk_finish<K, Q>(v, q, c0, a.vocab);
    probs_and_maps<K>(a, v, row, chunk, inv, prefix, rdraw, vec_out, ksum, s_first);
}

// ---- stages 1-3 in one launch (many rows) -----------------------------------
// As three launches, stages 1 and 2 each read the logits and stage 3 reads the
// exponentials that stage 2 wrote: each stage is a short kernel whose
// workgroups make a few dependent memory round trips, and the ramp and drain
// of every launch leave the GPU part idle.  Here each workgroup keeps its
// chunk in registers through all three stages (adjusted logits, then
// exponentials, then probabilities): the logits are read once and the
// probabilities written once.  The same operations on the same values give
// the same bits as the three launches.
//
// Between the stages the row's workgroups meet at a barrier.  A workgroup
// publishes its chunk maximum (then its chunk sum) with device-scope stores,
// waits for them to complete, and sets its done flag to this call's token;
// its first wave then polls the row's flags with device-scope loads (they
// bypass the per-XCD L2, which is not coherent across XCDs).  No counter
// takes the arrivals: arrivals on one address serialise at the memory side.
// The token is the workspace's epoch + 1, and the walk, which runs after
// every workgroup of this launch has finished, advances the epoch: flags
// never need clearing, and a flag left by an earlier call never matches.
// A barrier needs all of its row's workgroups resident at once, which the
// workgroup order below guarantees for the lowest unfinished row whatever
// else holds the GPU; the host takes this path only where the whole grid
// fits on the GPU at once, where it measured faster.  A wait still gives up
// after kRowWaitTicks of real time, marks its row (the walk then returns id
// -1 for it) and goes on, so every wave exits.
// Chunk sizes of the one launch, in k-slices (4096, 8192, 12288 logits per
// workgroup); the host takes the smallest whose grid fits on the GPU at once.
constexpr int kFusedKMin = 4;
constexpr uint64_t kRowWaitTicks = 20000000u;  // 0.2 s of s_memrealtime (100 MHz)

__device__ __forceinline__ uint64_t ld_agent(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_agent(const int32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 polls the n flags until every one holds tok (false after
// kRowWaitTicks); the workgroup's barrier then hands the answer to all.
__device__ bool row_wait(const uint64_t* flags, int n, uint64_t tok, int* s_ok) {
    if (threadIdx.x < kWave) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        bool ok = false;
        while (true) {
            bool mine = true;
            for (int c = threadIdx.x; c < n; c += kWave) mine = mine && ld_agent(flags + c) == tok;
            if (__all(mine)) {
                ok = true;
                break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > kRowWaitTicks) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (threadIdx.x == 0) *s_ok = ok ? 1 : 0;
    }
    __syncthreads();
    return *s_ok != 0;
}

// Registers: chunks of 12 k-slices at most 128 VGPRs (4 waves per SIMD), so
// that 4 workgroups fit on a CU (the cap also measured 1 us faster per call
// than the 121 VGPRs left to the compiler, 16 bytes of spill per lane);
// chunks of 8 at most 96 (5 per CU, no spill), so that 64 rows of 151936
// (1216 workgroups) fit on the GPU at once with them: 58.7 -> 53.4 us per
// call against chunks of 12 (at 80 VGPRs, 6 per CU, it spilled 56 bytes per
// lane and took 55.5-55.9); chunks of 4 take 68 (7 per CU) uncapped.
// Grid (nchunk, rows), chunks of K slices.  A row's workgroups are
// consecutive in dispatch order (blockIdx.x its chunk, blockIdx.y the row),
// so the launch makes progress however few of its workgroups are resident:
// workgroups are dispatched in order, so the lowest row not yet finished has
// all its workgroups dispatched (its at most a few dozen workgroups cannot
// fill the GPU's slots by themselves, and every lower row has finished and
// left its slots), finishes, and frees its slots for the next.  That covers
// a grid larger than the GPU holds and a GPU shared with other launches,
// e.g. another call on another stream.  (Chunk 0 of every row first, as in
// stage 3, measured 64.3 against 65.1 us at 64 rows, but with fewer
// workgroups resident than the grid no row would have all of its.)
template <int K>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(K == 8 ? 5 : 4))) void sample_fused_kernel(SampleArgs a, int vec, int vec_out) {
    constexpr int kCH = K * kSlice;
    __shared__ __align__(16) uint32_t cnt[kCH / 2];   // window counts, two per word
    __shared__ float red[4];
    __shared__ uint64_t red_s[4], red_p[4];
    __shared__ int red_f[4];
    __shared__ float ksum[K][4];
    __shared__ __align__(16) float s_first[kFirstN];
    __shared__ int s_ok[2];
    const long row = blockIdx.y;
    const int chunk = (int)blockIdx.x;
    const long c0 = (long)chunk * kCH;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    // The call's token: the epoch, which only the walk kernel (a later
    // launch) changes, so a plain load sees the last call's value; the load
    // goes out first, and the token is taken into scalar registers once the
    // chunk has arrived.
    const uint64_t epoch = *a.epoch;
    const float rdraw = a.r[row];
    float v[4 * K];
    float4 q[K];
    // A run-time choice of the load path, not a template parameter: with only
    // the quad path compiled in, the register allocation spilled inside the
    // exponentials (96 bytes per lane against 16).  Each path loads its own
    // window entry first (the empty asm statements keep the compiler from
    // hoisting that load out of both): the compiler's view of the branch
    // includes a path through neither, and an entry loaded before the branch
    // was the newest load on it, which made the count wait for every quad.
    const bool quads = chunk_quads(a.vocab, vec != 0);
    HistFirst hf;
    if (quads) {
        asm volatile("; quad path");
        hf = hist_first(a, row);
        __builtin_amdgcn_sched_barrier(0);
        load_chunk_issue<K, true>(q, v, a.logits + row * a.ld_logits, c0, a.vocab);
    } else {
        asm volatile("; element path");
        hf = hist_first(a, row);
        load_chunk_issue<K, false>(q, v, a.logits + row * a.ld_logits, c0, a.vocab);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int id0 = first_id(hf);
    build_counts<true>(cnt, kCH, a, row, c0, hf, id0);   // while the chunk is in flight
    if (quads) load_chunk_finish<K, true>(v, q, c0, a.vocab);
    const uint64_t tok = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(epoch >> 32)) << 32 |
                          (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)epoch)) + 1u;
    adjust_k<K, true>(v, cnt, a);
    const int nvalid = a.vocab - c0 < kCH ? (int)(a.vocab - c0) : kCH;
    uint64_t* flags1 = a.ws_tok + row * 2 * a.nchunk;
    uint64_t* flags2 = flags1 + a.nchunk;
    bool ok = true;

    // stage 1: the chunk maximum of the adjusted logits
    // A whole chunk, every chunk of a row but its last, takes no selects here
    // and in the exponentials: 64 rows of 151936, 63.2 -> 60.2 us per call
    // (the stages are bound by their vector instructions).
    float best = -INFINITY;
    if (nvalid == kCH) {
#pragma unroll
        for (int i = 0; i < 4 * K; i++) best = fmaxf(best, v[i]);
    } else {
#pragma unroll
        for (int k = 0; k < K; k++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                best = k * kSlice + 4 * (int)threadIdx.x + e < nvalid ? fmaxf(best, v[4 * k + e]) : best;
    }
    best = wave_max(best);
    if (lane == 0) red[wid] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        if (chunk == 0) st_agent(a.ws_rowtok + 2 * row, tok);
        st_agent(a.ws_max + row * a.nchunk + chunk, fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
        __builtin_amdgcn_s_waitcnt(0);   // the maximum has landed before the flag says so
        st_agent(flags1 + chunk, tok);
    }
    ok = row_wait(flags1, a.nchunk, tok, &s_ok[0]) && ok;
    float m = -INFINITY;
    for (int c = threadIdx.x; c < a.nchunk; c += blockDim.x) m = fmaxf(m, ld_agent(a.ws_max + row * a.nchunk + c));
    const float neg = -reduce_max(m, red);

    // stage 2: the exponentials, kept, and the chunk's exact sum
    constexpr int kLogTerms = K <= 4 ? 4 : K <= 8 ? 5 : 6;  // ceil(log2(4K)), a lane's terms
    static_assert(4 * K <= (1 << kLogTerms), "a lane's terms");
    uint64_t acc;
    int nan;
    const bool f64 = a.shift + kLogTerms <= 53;   // uniform: the lane's sum fits fp64's 53 bits
    if (nvalid == kCH) {
        if (f64) exp_and_sum_keep<K, true, true>(v, neg, a, nvalid, acc, nan);
        else exp_and_sum_keep<K, false, true>(v, neg, a, nvalid, acc, nan);
    } else {
        if (f64) exp_and_sum_keep<K, true, false>(v, neg, a, nvalid, acc, nan);
        else exp_and_sum_keep<K, false, false>(v, neg, a, nvalid, acc, nan);
    }
    acc = wave_sum_u64(acc);
    nan = __any(nan) ? 1 : 0;
    if (lane == 0) {
        red_s[wid] = acc;
        red_f[wid] = nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        st_agent(a.ws_sum + row * a.nchunk + chunk, red_s[0] + red_s[1] + red_s[2] + red_s[3]);
        st_agent(a.ws_flag + row * a.nchunk + chunk, red_f[0] | red_f[1] | red_f[2] | red_f[3]);
        __builtin_amdgcn_s_waitcnt(0);
        st_agent(flags2 + chunk, tok);
    }
    ok = row_wait(flags2, a.nchunk, tok, &s_ok[1]) && ok;
    if (!ok && threadIdx.x == 0) st_agent(a.ws_rowtok + 2 * row + 1, tok);   // the walk returns -1 for this row
    SumShare sh = {0u, 0u, 0};
    for (int c = threadIdx.x; c < a.nchunk; c += blockDim.x) {
        const uint64_t w = ld_agent(a.ws_sum + row * a.nchunk + c);
        sh.all += w;
        sh.pre += c < chunk ? w : 0u;
        sh.flag |= ld_agent(a.ws_flag + row * a.nchunk + c);
    }
    float inv, prefix;
    reduce_sums(sh, a, red_s, red_p, red_f, inv, prefix);

    // stage 3
    probs_and_maps<K>(a, v, row, chunk, inv, prefix, rdraw, vec_out, ksum, s_first);
}

// ---- the walk ------------------------------------------------------------------
// One wave per row; no barriers after the set-up.  The wave passes as many
// 256-probability sub-tiles at once as their stored maps allow and walks the
// others exactly, lane l owning elements 4l..4l+3 of the sub-tile (lane order
// is index order).  The probabilities are read back from the stage-3 output.
constexpr int kSumCache = 4096;  // sub-tile summaries cached in LDS per row
constexpr uint32_t kNoEv = 0xFFFFFFFFu;

constexpr int kXCache = 2048;  // sub-tiles whose crossing data is cached in LDS per row

struct __align__(16) WalkShared {
    uint32_t sm0[kSumCache], sm1[kSumCache];  // sub-tile maps
    int32_t scls[kSumCache];                   // predicted binade classes
    uint32_t xing[kXCache * kXWords];          // predicted crossings
};

// One memory round of the cache fill: K 16-byte loads per lane from a
// source of nq quads (16-byte aligned rows), every load issued before the
// first LDS store.  Loads and stores both use the clamped index, so neither
// sits behind a branch (a guarded store lets the compiler sink its load into
// the branch, one memory latency per quad); lanes past the end rewrite the
// last quad with its own value.  The source row stride is a multiple of 4
// words, so the last quad is in bounds; the LDS destination holds whole quads.
template <int K>
__device__ __forceinline__ void fill_round(const int4* src, int nq, int b, int4 t[K]) {
    const int lane = threadIdx.x;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int j = b + k * 64 + lane;
        t[k] = src[j < nq ? j : nq - 1];
    }
}
template <int K>
__device__ __forceinline__ void drain_round(int4* d, int nq, int b, const int4 t[K]) {
    const int lane = threadIdx.x;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int j = b + k * 64 + lane;
        d[j < nq ? j : nq - 1] = t[k];
    }
}

// The row's sub-tile summaries (maps and classes: nm sub-tiles; crossings:
// nx sub-tiles) from global memory to LDS by one wave.  At V = 151936 (594
// sub-tiles) everything arrives in one memory round trip.
__device__ void fill_walk_cache(WalkShared& sh, const SampleArgs& a, long row, int nm, int nx) {
    constexpr int KM = 4, KX = 16;  // quads per lane and round
    const int4* s0 = reinterpret_cast<const int4*>(a.ws_map0 + row * a.nsub_ld);
    const int4* s1 = reinterpret_cast<const int4*>(a.ws_map1 + row * a.nsub_ld);
    const int4* s2 = reinterpret_cast<const int4*>(a.ws_cls + row * a.nsub_ld);
    const int4* sx = reinterpret_cast<const int4*>(a.ws_xing + row * a.nsub_ld * kXWords);
    const int qm = (nm + 3) / 4, qx = (nx * kXWords + 3) / 4;
    int4 t0[KM], t1[KM], t2[KM], tx[KX];
    fill_round<KM>(s0, qm, 0, t0);
    fill_round<KM>(s1, qm, 0, t1);
    fill_round<KM>(s2, qm, 0, t2);
    fill_round<KX>(sx, qx, 0, tx);
    drain_round<KM>(reinterpret_cast<int4*>(sh.sm0), qm, 0, t0);
    drain_round<KM>(reinterpret_cast<int4*>(sh.sm1), qm, 0, t1);
    drain_round<KM>(reinterpret_cast<int4*>(sh.scls), qm, 0, t2);
    drain_round<KX>(reinterpret_cast<int4*>(sh.xing), qx, 0, tx);
    for (int b = 64 * KM; b < qm; b += 64 * KM) {  // larger vocabularies
        fill_round<KM>(s0, qm, b, t0);
        fill_round<KM>(s1, qm, b, t1);
        fill_round<KM>(s2, qm, b, t2);
        drain_round<KM>(reinterpret_cast<int4*>(sh.sm0), qm, b, t0);
        drain_round<KM>(reinterpret_cast<int4*>(sh.sm1), qm, b, t1);
        drain_round<KM>(reinterpret_cast<int4*>(sh.scls), qm, b, t2);
    }
    for (int b = 64 * KX; b < qx; b += 64 * KX) {
        fill_round<KX>(sx, qx, b, tx);
        drain_round<KX>(reinterpret_cast<int4*>(sh.xing), qx, b, tx);
    }
}

// Pass a crossing sub-tile in O(1) from the exact running sum at its start
// (bits cb) with its stored crossing x (the kXWords words) and predicted
// class pcls, if every stored prediction holds: the sum starts in the binade
// pre was made for and stays in it up to element j, leaves it at j, the fp32
// sum after j lies in the binade the suffix map was made for and stays there,
// and no running sum reaches r.  Returns false (nothing changed) otherwise;
// the caller then walks the sub-tile exactly.  Straight-line: every check is
// evaluated (on wave-uniform values) and decided once at the end.
__device__ __forceinline__ bool pass_crossing(uint32_t& cb, const uint32_t (&x)[kXWords], int pcls, float r) {
    const int info = (int)x[5];
    if (info < 0) return false;   // no single crossing predicted (uniform: a scalar branch)
    const Binade b = binade_of(__uint_as_float(cb));
    const uint32_t inc = pick(Fn{x[0], x[1]}, b.m0);  // arithmetic select: an indexed one went to scratch
    const uint32_t mb = b.m0 + inc;  // m0 < 2^24, inc <= 2^30: no wrap
    const float base = ldexpf((float)mb, -b.sh);
    const float pj = __uint_as_float(x[4]);
    const uint32_t incj = pick(elem_map(pj, b), mb);
    const float c = base + pj;  // the reference's fp32 add of element j
    const Binade b2 = binade_of(c);
    const uint32_t inc2 = pick(Fn{x[2], x[3]}, b2.m0);
    const float end = ldexpf((float)(b2.m0 + inc2), -b2.sh);
    const bool ok = (info >= 0) & (b.cls == pcls)                // a single crossing, made for this binade
                    & (inc < b.mhi - b.m0) & (base < r)           // no leave and no hit before j
                    & !(incj < b.mhi - mb) & (c < r)              // leaves at j; the draw does not end there (nor NaN)
                    & (b2.cls == (info >> 8)) & (inc2 < b2.mhi - b2.m0) & (end < r);  // the rest stays, no hit
    if (ok) cb = __float_as_uint(end);
    return ok;
}

// Exact walk of sub-tile st from the running sum with bits cb.  Inside one
// binade the running sums of all 256 elements follow from one in-order wave
// scan of their maps; an element that leaves the binade is added with an
// ordinary fp32 add and the scan restarts after it.  Returns true when the
// draw is decided (result set), else updates cb to the sub-tile's end.
// The first nsubs sub-tiles (elements 0 .. min(V, 256 * nsubs) - 1, nsubs <=
// kFirstSubs) one fp32 add at a time in index order, from cum = 0: the
// reference's loop itself, run by one lane over the probabilities staged in
// LDS (sp, 16-byte aligned).  Returns
// true when the draw is decided (result set), else sets cb to the running
// sum's bits at their end.  Adding 0.0f for the padding past V leaves the sum
// unchanged.
// The 16 running sums after cum, in index order, and whether the draw ends
// among them (result set).  One fp32 add per element, as the reference.
__device__ __forceinline__ bool walk16(const float4 (&q)[4], int i, long V, float r, float& cum, long& result) {
    float c[16];
    float run = cum;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        run = run + q[u].x;
        c[4 * u] = run;
        run = run + q[u].y;
        c[4 * u + 1] = run;
        run = run + q[u].z;
        c[4 * u + 2] = run;
        run = run + q[u].w;
        c[4 * u + 3] = run;
    }
    if (!(c[15] < r)) {  // the draw ends in these 16, or the sum became NaN (cum never decreases)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            if (c[e] >= r) {
                result = i + e;
                return true;
            }
            if (c[e] != c[e]) {  // no later sum can reach r
                result = V - 1;
                return true;
            }
        }
    }
    cum = c[15];
    return false;
}

__device__ bool walk_first_lds(const float* sp, int nsubs, long V, float r, uint32_t& cb, long& result) {
    const int nel = nsubs * kSub;
    const int nvalid = V < nel ? (int)V : nel;
    float cum = 0.0f;
    if (nvalid == nel) {
        // whole sub-tiles: no per-element bounds, and the next 16
        // probabilities are read from LDS while these 16 are added
        float4 q[4], nq[4];
#pragma unroll
        for (int u = 0; u < 4; u++) q[u] = *reinterpret_cast<const float4*>(sp + 4 * u);
        for (int i = 0; i < nel; i += 16) {
            const int n = i + 16 < nel ? i + 16 : i;
#pragma unroll
            for (int u = 0; u < 4; u++) nq[u] = *reinterpret_cast<const float4*>(sp + n + 4 * u);
            if (walk16(q, i, V, r, cum, result)) return true;
#pragma unroll
            for (int u = 0; u < 4; u++) q[u] = nq[u];
        }
        cb = __float_as_uint(cum);
        return false;
    }
    for (int i = 0; i < nvalid; i += 16) {
        float4 q[4];
#pragma unroll
        for (int u = 0; u < 4; u++) q[u] = *reinterpret_cast<const float4*>(sp + i + 4 * u);
        float c[16];
        float run = cum;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float e4[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                run = run + (i + 4 * u + e < nvalid ? e4[e] : 0.0f);
                c[4 * u + e] = run;
            }
        }
        if (!(c[15] < r)) {  // the draw ends in these 16, or the sum became NaN (cum never decreases)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                if (i + e < nvalid) {
                    if (c[e] >= r) {
                        result = i + e;
                        return true;
                    }
                    if (c[e] != c[e]) {  // no later sum can reach r
                        result = V - 1;
                        return true;
                    }
                }
            }
        }
        cum = c[15];
    }
    cb = __float_as_uint(cum);
    return false;
}

// p: this lane's four probabilities of the sub-tile starting at index base
// (elements base + 4*lane ..); one wave.
__device__ bool walk_subtile_p(const float p[4], long base, long V, float r, uint32_t& cb, long& result) {
    const int lane = threadIdx.x & 63;
    // offsets inside the sub-tile: first unprocessed element, end of the row
    const int nvalid = V - base < kSub ? (int)(V - base) : kSub;
    int s = 0;
    while (true) {
        const Binade b = binade_of(__uint_as_float(cb));
        Fn f[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int o = 4 * lane + e;
            const Fn m = elem_map(p[e], b);
            const bool in = o >= s && o < nvalid;
            f[e].a0 = in ? m.a0 : 0u;
            f[e].a1 = in ? m.a1 : 0u;
        }
        const Fn incl = compose4_scan(f);
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

__device__ bool walk_subtile(const SampleArgs& a, long st, const float* prow, float r, uint32_t& cb, long& result) {
    const int lane = threadIdx.x & 63;
    const long V = a.vocab;
    const long i0 = st * kSub + 4 * lane;
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
    return walk_subtile_p(p, st * kSub, V, r, cb, result);
}

// one wave per row and per CU: all of the register file is available to it
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void sample_walk_kernel(SampleArgs a) {
    __shared__ WalkShared sh;
    const int lane = threadIdx.x;
    const long row = blockIdx.x;
    // After a one-launch call: the next call's token is one more, and a row
    // whose barrier gave up in that launch has no valid draw.  The tokens were
    // written by that launch, so plain loads see them; they go out with the
    // cache fill's loads, unconditionally (after three launches they read a
    // chunk sum instead), and are compared after it.
    if (a.epoch && row == 0 && lane == 0)
        __hip_atomic_fetch_add(a.epoch, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t* tp = a.epoch ? a.ws_rowtok + 2 * row : a.ws_sum + row * a.nchunk;
    const uint64_t tok0 = tp[0], tok1 = tp[a.epoch ? 1 : 0];
    const float r = a.r[row];
    const long V = a.vocab;
    const float* prow = a.probs + row * a.ld_probs;
    const int first_hit = a.ws_first[2 * row];  // sub-tiles 0..first_subs-1, walked by stage 3
    const uint32_t first_end = (uint32_t)a.ws_first[2 * row + 1];
    const int ncache = a.nsub < kSumCache ? a.nsub : kSumCache;
    const int nxcache = a.nsub < kXCache ? a.nsub : kXCache;
    fill_walk_cache(sh, a, row, ncache, nxcache);
    __syncthreads();
    if (a.epoch && tok0 == tok1) {
        if (lane == 0) a.ids[row] = -1;
        return;
    }
    // "cum < r" on bit patterns: cum >= 0, so cum < r <=> bits(cum) < bits(r)
    // for r > 0; for r <= 0 or NaN no sub-tile is passed without a walk
    const uint32_t rb = r > 0.0f ? __float_as_uint(r) : 0u;
    if (first_hit >= 0) {
        if (lane == 0) a.ids[row] = first_hit;
        return;
    }
    uint32_t cb = first_end;  // bits of the running sum
    long result = V - 1;
    long st = a.first_subs;
    // every record of the row in LDS (V <= 2048 sub-tiles): each step reads
    // its 64 sub-tiles' class, map and crossing in one round of LDS loads
    const bool all_cached = a.nsub <= nxcache;
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
        int lcls = -1;                   // this lane's predicted class
        uint32_t lx[kXWords] = {0u, 0u, 0u, 0u, 0u, 0xFFFFFFFFu};  // and crossing (all_cached)
        if (all_cached) {  // row-uniform; unconditional loads at a clamped index
            const int ic = idx < a.nsub ? (int)idx : a.nsub - 1;
            lcls = sh.scls[ic];
            const uint32_t s0 = sh.sm0[ic], s1 = sh.sm1[ic];
            const uint2* xp = reinterpret_cast<const uint2*>(&sh.xing[ic * kXWords]);
#pragma unroll
            for (int w = 0; w < kXWords / 2; w++) {
                const uint2 q = xp[w];
                lx[2 * w] = q.x;
                lx[2 * w + 1] = q.y;
            }
            const bool use = idx < a.nsub && lcls == ccls;
            f.a0 = use ? s0 : kSat;
            f.a1 = use ? s1 : kSat;
        } else if (idx < a.nsub) {
            const int pc = idx < kSumCache ? sh.scls[idx] : a.ws_cls[row * a.nsub_ld + idx];
            if (pc == ccls) {
                f.a0 = idx < kSumCache ? sh.sm0[idx] : a.ws_map0[row * a.nsub_ld + idx];
                f.a1 = idx < kSumCache ? sh.sm1[idx] : a.ws_map1[row * a.nsub_ld + idx];
            }
        }
        const Fn pre = wave_scan_any(f);
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
            // a predicted crossing passes in O(1); anything else is walked
            // exactly.  A stop whose map stays in the binade is the draw
            // ending inside that map, which no crossing record can pass.
            bool passed = false;
            const bool leaves = !((uint32_t)__builtin_amdgcn_readlane((int)inc, npass) < mhi - m0);
            if (!leaves) {
            } else if (all_cached) {  // the stopping lane's record, already loaded
                uint32_t x[kXWords];
#pragma unroll
                for (int w = 0; w < kXWords; w++) x[w] = (uint32_t)__builtin_amdgcn_readlane((int)lx[w], npass);
                passed = pass_crossing(cb, x, __builtin_amdgcn_readlane(lcls, npass), r);
            } else if (st < nxcache) {
                uint32_t x[kXWords];
#pragma unroll
                for (int w = 0; w < kXWords; w++) x[w] = sh.xing[st * kXWords + w];
                const int pc = st < kSumCache ? sh.scls[st] : a.ws_cls[row * a.nsub_ld + st];
                passed = pass_crossing(cb, x, pc, r);
            }
            if (!passed && walk_subtile(a, st, prow, r, cb, result)) break;
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
    size_t off_epoch, off_rowtok, off_tok, off_sum, off_max, off_arg, off_flag, off_m0, off_m1, off_cls, off_x,
        off_first, total;
};

static size_t al16(size_t x) { return (x + 15) & ~(size_t)15; }

// 1024-logit slices per chunk of the three launches: 1 up to about 14
// workgroups of 1024 logits per CU (24 rows of 151936), else 3.  The
// stages' per-wave work is a chain of dependent instructions over a
// thread's 4K logits and a wave's K sub-tiles, so smaller chunks finish
// sooner until the grid is many rounds deep.  Per call at 151936 (8 calls on
// distinct inputs per graph), chunks of 1 against 3: 7 rows 31.9 / 41.2 us,
// 12 rows 37.2 / 42.8, 16 rows 43.2 / 47.2, 24 rows 52.9 / 53.6 (unaligned
// probabilities), 32 rows 59.4 / 56.6; at 64 rows 3 measured 68.5 us against
// 70.7 for 4, 73-75 for 2 and 73-81 for 5, 6 and 8.  The outputs do not
// depend on it.
constexpr int kSlicesMany = 3;
static int chunk_slices(long rows, long vocab) {
    return rows * ((vocab + kSlice - 1) / kSlice) < 3600 ? 1 : kSlicesMany;
}

static WsLayout ws_layout(long rows, long vocab) {
    const long kch = (long)chunk_slices(rows, vocab) * kSlice;
    const size_t nch = (size_t)((vocab + kch - 1) / kch);
    const size_t nsub = (size_t)((vocab + kSub - 1) / kSub);
    const size_t n = (size_t)rows * nch, ns = (size_t)rows * ((nsub + 3) & ~(size_t)3);
    // the one launch's flags, for its smallest chunks (the most per row); its
    // chunk maxima and sums use the regions below, which hold a chunk of 3
    // k-slices or fewer per entry
    const size_t nchf = (size_t)((vocab + kFusedKMin * kSlice - 1) / (kFusedKMin * kSlice));
    WsLayout l;
    // the one-launch path's epoch first, at the same place for every shape
    // (it counts the calls made on the workspace, whatever their shapes)
    l.off_epoch = 0;
    l.off_rowtok = 256;
    l.off_tok = l.off_rowtok + al16((size_t)rows * 2 * sizeof(uint64_t));
    l.off_sum = l.off_tok + al16((size_t)rows * 2 * nchf * sizeof(uint64_t));
    l.off_max = l.off_sum + al16(n * sizeof(uint64_t));
    l.off_arg = l.off_max + al16(n * sizeof(float));
    l.off_flag = l.off_arg + al16(n * sizeof(int32_t));
    l.off_m0 = l.off_flag + al16(n * sizeof(int32_t));
    l.off_m1 = l.off_m0 + al16(ns * sizeof(uint32_t));
    l.off_cls = l.off_m1 + al16(ns * sizeof(uint32_t));
    l.off_x = l.off_cls + al16(ns * sizeof(int32_t));
    l.off_first = l.off_x + al16(ns * kXWords * sizeof(uint32_t));
    l.total = l.off_first + al16((size_t)rows * 2 * sizeof(int32_t));
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
    a.ws_xing = reinterpret_cast<uint32_t*>(b + l.off_x);
    a.ws_first = reinterpret_cast<int32_t*>(b + l.off_first);
    a.ws_tok = nullptr;   // set by the one-launch path
    a.ws_rowtok = nullptr;
    a.epoch = nullptr;
    const long kch = (long)chunk_slices(rows, vocab) * kSlice;
    a.nchunk = (int)((vocab + kch - 1) / kch);
    a.nsub = (int)((vocab + kSub - 1) / kSub);
    a.nsub_ld = (a.nsub + 3) & ~3;
    a.first_subs = chunk_slices(rows, vocab) == 1 ? 1 : kFirstSubs;
    a.shift = 63 - ceil_log2(vocab);
    // the sequential fp32 running sum of vocab probabilities is within
    // vocab * 2^-25 of the exact prefix (each add errs by half an ulp of a
    // sum below 1), plus slack for the prediction's own rounding
    a.skip_margin = (float)((double)vocab * 0x1p-25 + 0x1p-10);
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

namespace anelm {
namespace {
// Stages 1-3 (the quad paths chosen per input: logits for stages 1 and 2,
// the stored exponentials for stage 3).
template <int K>
void launch_stages(const SampleArgs& a, dim3 grd, bool q_in, bool q_out, int vec_out, hipStream_t st) {
    if (q_in) {
        sample_stage1_kernel<false, K, true><<<grd, 256, 0, st>>>(a);
        sample_stage2_kernel<K, true><<<grd, 256, 0, st>>>(a, vec_out);
    } else {
        sample_stage1_kernel<false, K, false><<<grd, 256, 0, st>>>(a);
        sample_stage2_kernel<K, false><<<grd, 256, 0, st>>>(a, vec_out);
    }
    if (q_out) sample_stage3_kernel<K, true><<<grd, 256, 0, st>>>(a, vec_out);
    else sample_stage3_kernel<K, false><<<grd, 256, 0, st>>>(a, vec_out);
}
}  // namespace
}  // namespace anelm

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
    const bool q = chunk_quads(n, vec != 0);
    const dim3 grd((unsigned)a.nchunk, (unsigned)rows);
    if (chunk_slices(rows, n) == 1) launch_stages<1>(a, grd, q, q, vec, st);
    else launch_stages<kSlicesMany>(a, grd, q, q, vec, st);
    return launch_status("softmax");
}

namespace anelm {
namespace {

// The one-launch path from this many rows.  Per call at 151936 logits (8
// calls on distinct inputs in a graph), one launch (chunks of 4 k-slices)
// against three (chunks of 1): 6 rows 33.3 / 30.7 us, 8 rows 36.1 / 33.2, 10
// rows 35.7 / 35.3, 12 rows 36.2 / 37.2, 16 rows 38.8 / 43.2.
constexpr long kFusedMinRows = 12;
// Sub-tiles that chunk 0 of each row walks one add at a time in the one
// launch.  There every workgroup finishes at about the same time, so this
// walk (about 8 cycles an add) lengthens the launch, where stage 3 of the
// three launches hid it; what it leaves to the walk costs there instead.
// Per call at 64 rows (one launch + walk, under the profiler): 0 sub-tiles
// 43.0 + 20.5 us, 1: 42.9 + 15.5, 2: 43.1 + 14.4, 4: 45.7 + 14.0.
constexpr int kFusedFirstSubs = 2;
constexpr int kCapDevices = 64;

// Workgroups of the one-launch kernel with chunks of K k-slices that the
// current device holds at once (occupancy per CU x CUs), looked up once per
// device; 0 if unknown.
template <int K>
long fused_capacity() {
    static std::mutex mu;
    static long cap[kCapDevices];
    static bool known[kCapDevices];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kCapDevices) return 0;
    std::lock_guard<std::mutex> lock(mu);
    if (!known[dev]) {
        int nb = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, sample_fused_kernel<K>, 256, 0) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
            (void)hipGetLastError();
            nb = cus = 0;
        }
        cap[dev] = (long)nb * cus;
        known[dev] = true;
    }
    return cap[dev];
}

// Fits in 95% of what the GPU holds at once (85% with chunks of 4 k-slices:
// 44 rows of 151936 at 93% of their capacity took 56.8 us per call against
// 49.1 with chunks of 8, 40 rows at 85% 46.9 us).
template <int K>
bool fused_fits(long rows, long vocab) {
    const long nchf = (vocab + K * kSlice - 1) / (K * kSlice);
    return rows * nchf * 20 <= fused_capacity<K>() * (K == 4 ? 17 : 19);
}

// The one launch's chunk size in k-slices for a sampling call, or 0 for the
// three launches: many rows, aligned rows (16-byte loads and stores
// throughout), a window short enough for 16-bit counts, and the smallest
// chunks whose grid fits on the GPU at once with room to spare (fused_fits;
// for speed: the launch completes without that too, row after row).  Smaller chunks put
// more of the GPU on the rows and shorten each workgroup's chain; per call at
// 151936 logits (8 calls on distinct inputs per graph), chunks of 4 / 8 / 12
// k-slices: 32 rows 42.7 / 46.1 / 50.5 us, 48 rows (4 does not fit) 50.0 /
// 55.5, 64 rows (8 at 5 workgroups per CU) 53.4 / 58.7.
int fused_k(long rows, long vocab, long hist_ld, int ctx, bool penalty, int vec, int vec_out) {
    if (rows < kFusedMinRows || !vec || !vec_out) return 0;
    if (penalty && (ctx < hist_ld ? (long)ctx : hist_ld) > 65535) return 0;
    if (fused_fits<4>(rows, vocab)) return 4;
    if (fused_fits<8>(rows, vocab)) return 8;
    if (fused_fits<12>(rows, vocab)) return 12;
    return 0;
}

// The sampler behind both entry points; `who` names the caller in errors.
int sample_impl(int32_t* ids, float* probs, long ld_probs, const float* logits, long ld_logits, long rows, long vocab,
                const int32_t* hist, long hist_ld, const int32_t* hist_len, const anelm_sampling_params* params,
                const float* r, void* workspace, size_t workspace_bytes, void* stream, const char* who) {
    if (!ids || !logits || !params) return fail(ANELM_ERR_INVALID, "%s: null pointer", who);
    if (rows <= 0 || rows > 65535 || vocab <= 0 || vocab > (1L << 30))
        return fail(ANELM_ERR_INVALID, "%s: rows=%ld vocab=%ld", who, rows, vocab);
    if (ld_logits < vocab) return fail(ANELM_ERR_INVALID, "%s: ld_logits < vocab", who);
    if (probs && ld_probs < vocab) return fail(ANELM_ERR_INVALID, "%s: ld_probs < vocab", who);
    if (hist_ld < 0 || (hist_ld > 0 && !hist)) return fail(ANELM_ERR_INVALID, "%s: history", who);
    const bool sampling = params->temperature > 0.0f;
    if (sampling && !r) return fail(ANELM_ERR_INVALID, "%s: r is required when temperature > 0", who);
    if (sampling && !probs) return fail(ANELM_ERR_INVALID, "%s: probs is required when temperature > 0", who);
    SampleArgs a = {};
    int rc = bind_workspace(a, workspace, workspace_bytes, rows, vocab, who);
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
    const bool one = chunk_slices(rows, vocab) == 1;
    const bool q_in = chunk_quads(vocab, vec != 0);
    if (!sampling) {
        if (one) {
            if (q_in) sample_stage1_kernel<true, 1, true><<<grd, 256, 0, st>>>(a);
            else sample_stage1_kernel<true, 1, false><<<grd, 256, 0, st>>>(a);
        } else {
            if (q_in) sample_stage1_kernel<true, kSlicesMany, true><<<grd, 256, 0, st>>>(a);
            else sample_stage1_kernel<true, kSlicesMany, false><<<grd, 256, 0, st>>>(a);
        }
        sample_argmax_final_kernel<<<dim3((unsigned)rows), 64, 0, st>>>(a);
        return launch_status("sample(argmax)");
    }
    const int vec_out = probs && (ld_probs % 4 == 0) && aligned16(probs);
    a.vec_probs = vec_out;
    if (const int fk = fused_k(rows, vocab, hist_ld, a.ctx, a.use_penalty != 0, vec, vec_out)) {
        char* b = static_cast<char*>(workspace);
        const WsLayout l = ws_layout(rows, vocab);
        a.epoch = reinterpret_cast<uint64_t*>(b + l.off_epoch);
        a.ws_rowtok = reinterpret_cast<uint64_t*>(b + l.off_rowtok);
        a.ws_tok = reinterpret_cast<uint64_t*>(b + l.off_tok);
        a.nchunk = (int)((vocab + fk * kSlice - 1) / (fk * kSlice));
        a.first_subs = kFusedFirstSubs;
        const dim3 g((unsigned)a.nchunk, (unsigned)rows);
        if (fk == 4) sample_fused_kernel<4><<<g, 256, 0, st>>>(a, vec, vec_out);
        else if (fk == 8) sample_fused_kernel<8><<<g, 256, 0, st>>>(a, vec, vec_out);
        else sample_fused_kernel<12><<<g, 256, 0, st>>>(a, vec, vec_out);
    } else {
        const bool q_out = chunk_quads(vocab, vec_out != 0);
        if (one) launch_stages<1>(a, grd, q_in, q_out, vec_out, st);
        else launch_stages<kSlicesMany>(a, grd, q_in, q_out, vec_out, st);
    }
    sample_walk_kernel<<<dim3((unsigned)rows), 64, 0, st>>>(a);
    return launch_status("sample");
}

// ---- the allocation-free sampler's scratch ---------------------------------
// The sampler's workspace as a static device array: every GPU the library
// runs on holds its own copy (kScratchBytes) until the process ends.  Host
// code never passes the array's name to a kernel or a copy (on the host it
// is only a stand-in symbol): each device's address is looked up once with
// hipGetSymbolAddress, with that device current, and kept in scratch_ptr.
// Nothing in it needs clearing: every word a kernel reads is written earlier
// in the same call, except the one-launch path's epoch and flags, which work
// from any contents.  Calls that overlap on one GPU share it, and race.
constexpr size_t kScratchBytes = 4u << 20;   // 181 rows at Qwen3's 151936-row vocabulary
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
void* scratch_ptr[kMaxDevices];
std::mutex scratch_mu;

// this device's scratch address (looked up on its first call), or nullptr
// with the error set
void* device_scratch(const char* who) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        fail(ANELM_ERR_HIP, "%s: no usable current device (%d)", who, dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fail(ANELM_ERR_HIP, "%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", who, dev,
                 hipGetErrorString(e));
            return nullptr;
        }
        scratch_ptr[dev] = p;
    }
    return scratch_ptr[dev];
}

}  // namespace
}  // namespace anelm

extern "C" int anelm_sample(int32_t* ids, float* probs, long ld_probs, const float* logits, long ld_logits,
                            long rows, long vocab, const int32_t* hist, long hist_ld, const int32_t* hist_len,
                            const anelm_sampling_params* params, const float* r, void* workspace,
                            size_t workspace_bytes, void* stream) {
    return sample_impl(ids, probs, ld_probs, logits, ld_logits, rows, vocab, hist, hist_ld, hist_len, params, r,
                       workspace, workspace_bytes, stream, "anelm_sample");
}

extern "C" int anelm_sample_noalloc(int32_t* ids, float* probs, long ld_probs, const float* logits, long ld_logits,
                                    long rows, long vocab, const int32_t* hist, long hist_ld, const int32_t* hist_len,
                                    const anelm_sampling_params* params, const float* r, void* stream) {
    clear_error();
    if (rows > 0 && vocab > 0 && rows <= 65535 && vocab <= (1L << 30) && ws_layout(rows, vocab).total > kScratchBytes)
        return fail(ANELM_ERR_WORKSPACE,
                    "anelm_sample_noalloc: %ld rows x %ld logits need %zu bytes of scratch; the static scratch holds "
                    "%zu (use anelm_sample with a workspace)",
                    rows, vocab, ws_layout(rows, vocab).total, kScratchBytes);
    void* ws = device_scratch("anelm_sample_noalloc");
    if (!ws) return ANELM_ERR_HIP;
    return sample_impl(ids, probs, ld_probs, logits, ld_logits, rows, vocab, hist, hist_ld, hist_len, params, r, ws,
                       kScratchBytes, stream, "anelm_sample_noalloc");
}
