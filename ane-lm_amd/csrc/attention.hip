// GQA decode attention over per-sequence KV rings, and the ring append, for
// gfx950.  Replaces ane_lm::gqa_attention (core/cpu_ops.cpp:173-240) and the
// ring bookkeeping + row copies of models/llm/qwen3.cpp:475-488.
//
// Data layout: for sequence b the caches are k_cache/v_cache +
// b*cache_seq_stride, each [capacity, n_kv_heads, head_dim] fp32 (the
// reference's per-layer KVCache layout, qwen3.cpp:227-231).  The live rows
// are positions start, start+1, ... (mod capacity), len of them.
//
// Decode attention is HBM-bound on the cache: each K and V row of a kv head
// is read once and shared by all q heads of its group.  A workgroup owns one
// (sequence, kv head, chunk of <= 512 ring positions):
//   phase 1: 16 lanes per position (head_dim 128) hold 8 floats each of the
//            K row; dots for all group heads, reduced in-row with DPP;
//   phase 2: chunk softmax numerators (max, exp, sum) in LDS;
//   phase 3: the same position mapping over V rows, weighted accumulation.
// With one chunk per sequence the workgroup writes the normalised output;
// otherwise each chunk writes (max, sum, unnormalised output) partials and
// counts itself done, and the last chunk of a (sequence, kv head) to finish
// merges them.  The grid is (kv head, sequence, chunk), chunk slowest: a
// short ring is done by its chunk 0 alone (the other chunks exit at once), and
// with chunks dispatched last those workgroups all start in the first round.
// With many (sequence, kv head) pairs and rings of at most 2048 rows, one
// workgroup per pair takes the whole ring instead (the same phases over up
// to 2048 positions), and nothing is merged.
#include "anelm_common.hpp"

namespace anelm {
namespace {

constexpr int kAttnThreads = 256;     // 4 waves
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kMaxChunk = 512;        // ring positions per workgroup of a split launch
// Whole-ring launches: with at least kWholeRingPairs (sequence, kv head)
// pairs (two per CU) and rings of at most kWholeRingMax rows, one workgroup
// per pair attends over the whole ring and writes the output itself: no
// partials, counts or merges, whose tail latency in every split workgroup
// (device-scope stores, a count, the last chunk's loads) left its CU idle.
// 64 sequences at 8B shapes with 2048-row rings: 175 -> 165 us.  Below two
// pairs per CU some CUs would run two rings and others one.
constexpr int kWholeRingMax = 2048;
constexpr long kWholeRingPairs = 512;
// 64, not 32: a workgroup keeps two 32-position batches of loads in flight,
// so a 64-position chunk costs about one memory round trip like a 32-position
// one, and a long ring at a small batch has half the chunks to merge.
constexpr int kMinChunk = 64;
constexpr int kMaxGD = 1024;          // group heads x head_dim per workgroup
constexpr long kTargetBlocks = 2048;  // 8 workgroups per CU on 256 CUs
constexpr int kMaxSplit = 4096;       // chunks per sequence (capacity <= 4096*32)
constexpr int kWholeRows = 128;       // rings up to this long (or one chunk) are done by one workgroup
static_assert(kWholeRows <= kMaxChunk, "a whole ring's scores fit the LDS rows");

struct AttnArgs {
    float* out;
    uint16_t* out16;            // when set, outputs go here as fp16 (nearest even) instead of to out
    int out_cols;               // > 0: out16 in the tiled layout of anelm_proj_tile_f16, this many columns
    const float* q;
    const float* kc;
    const float* vc;
    const int32_t* ring_start;  // [batch] or null (then start0)
    const int32_t* ring_len;    // [batch] or null (then len0)
    int start0, len0;
    int nh, nkv, groups;
    long q_ld;                  // between sequences (elements)
    int q_hs;                   // between q heads
    long out_ld;                // between sequences; heads are head_dim apart
    int cap;
    long seq_stride;            // between sequences' caches
    int chunk, nsplit;
    int whole;                  // split launches: rings of at most this many rows are done by chunk 0 alone
    int g0, gcount;             // q heads g0 .. g0+gcount-1 of every group
    float scale;
    float* ws;                  // [batch*nh][nsplit][head_dim + 2] partials
    unsigned* ctr;              // [batch*nkv] chunks done (split launches; zero between launches)
    // QK launches (head_dim 128): q (at q, q_ld, q_hs = 128) and the new k and
    // v rows are the raw projection outputs.  q is normalised and rotated on
    // the fly; the workgroup whose chunk holds the ring's newest row (the
    // rings were advanced before the launch) makes that row from k and v and
    // writes it to the caches.
    const float* kraw;
    const float* vraw;
    long k_ld, v_ld;
    const void* wq;
    const void* wk;
    const int32_t* pos;
    const float* cos_tab;
    const float* sin_tab;
    int tab_len;
    float eps;
    float inv[64];              // RoPE inverse frequencies of the 64 pairs
    int whole_ring;             // launch one workgroup per (sequence, kv head) over the whole ring
};

// An attention output (sequence b, column col = head*head_dim + d): fp32, or
// fp16 rounded to nearest even (the input rounding of the projection that
// follows, done once here), in rows or in the tiled layout.
__device__ __forceinline__ void put_out(const AttnArgs& a, long b, int col, float v) {
    if (a.out16) {
        const long i = a.out_cols > 0 ? tiled_index(b, col, a.out_cols) : b * a.out_ld + col;
        a.out16[i] = __builtin_bit_cast(uint16_t, to_f16(v));
    } else {
        a.out[b * a.out_ld + col] = v;
    }
}

// The ring state of sequence b, clamped so that every access stays inside
// the caches: 0 <= len <= cap, 0 <= start < cap.
__device__ __forceinline__ void ring_state(const AttnArgs& a, long b, int& start, int& len) {
    int s = a.ring_start ? a.ring_start[b] : a.start0;
    int l = a.ring_len ? a.ring_len[b] : a.len0;
    l = l < 0 ? 0 : (l > a.cap ? a.cap : l);
    s %= a.cap;
    if (s < 0) s += a.cap;
    start = s;
    len = l;
}

// Ring slot of chunk position t (clamped to the chunk's last position n-1,
// n >= 1): start < cap and t0 + t < len <= cap, so one wrap suffices.
__device__ __forceinline__ int ring_slot(const AttnArgs& a, int start, int t0, int t, int n) {
    int slot = start + t0 + (t < n ? t : n - 1);
    if (slot >= a.cap) slot -= a.cap;
    return slot;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of LP lanes (8, 16 or 32); every lane of a group
// receives the same value.
template <int LP>
__device__ __forceinline__ float lp_sum(float v) {
    v += dpp<0xB1>(v);                       // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);                       // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);                      // row_half_mirror: the other quad
    if (LP >= 16) v += dpp<0x140>(v);        // row_mirror: the other 8 lanes
    if (LP >= 32) v += __shfl_xor(v, 16);
    return v;
}

// A lane's 8 elements of a head row: 4 at p[0..3] and 4 at p[D/2..D/2+3],
// with p = row + 4*ds, so that each load instruction of a lane group covers
// one contiguous half row.  NT: streamed once (non-temporal).
template <int D, bool NT>
__device__ __forceinline__ void load8(float (&x)[8], const float* p) {
    const float4* a4 = reinterpret_cast<const float4*>(p);
    const float4* b4 = reinterpret_cast<const float4*>(p + D / 2);
    const float4 a = NT ? ld_nt(a4) : *a4;
    const float4 b = NT ? ld_nt(b4) : *b4;
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merges the partials of chunks 0 .. live-1 of one (sequence, q head): one
// wave; lane j owns chunks j, j+64, ... for the (max, sum) merge, then every
// lane sums its head_dim/64 outputs over the chunks in chunk order.  The
// first kBatch chunks' output partials are loaded together with the (max,
// sum) pairs, before the max is known, so a ring of up to kBatch chunks costs
// one memory round trip.  Loads use clamped indices (chunk live-1 re-read,
// then discarded) so none sits behind a branch.  An empty chunk (sum 0)
// contributes nothing; NaN sums propagate.
template <int D>
__device__ void merge_head(const AttnArgs& a, long b, int h, int lane, int live) {
    constexpr int kBatch = D <= 128 ? 32 : 16;  // chunks whose partials are in flight at once
    const int ns = a.nsplit;
    const float* p = a.ws + (b * a.nh + h) * ns * (long)(D + 2);
    auto clampc = [&](int s) { return s < live ? s : live - 1; };
    // lane j holds chunk j's (max, sum); the first 64 stay in registers
    const float m0r = ld_dev(p + clampc(lane) * (D + 2) + D);
    const float l0r = ld_dev(p + clampc(lane) * (D + 2) + D + 1);
    float v[kBatch][D / kWave];
#pragma unroll
    for (int j = 0; j < kBatch; j++)
#pragma unroll
        for (int i = 0; i < D / kWave; i++) v[j][i] = ld_dev(p + clampc(j) * (D + 2) + lane + i * kWave);
    const float m0 = lane < live ? m0r : -INFINITY;
    const float l0 = lane < live ? l0r : 0.0f;
    float M = l0 > 0.0f ? m0 : -INFINITY;
    for (int s = lane + kWave; s < live; s += kWave) {
        if (ld_dev(p + s * (D + 2) + D + 1) > 0.0f) M = fmaxf(M, ld_dev(p + s * (D + 2) + D));
    }
    M = wave_max_rows(M);
    float L = 0.0f;
    float o[D / kWave];
#pragma unroll
    for (int i = 0; i < D / kWave; i++) o[i] = 0.0f;
    for (int s0 = 0; s0 < live; s0 += kWave) {
        const int s = s0 + lane;
        float ms = m0, ls = l0;
        if (s0 > 0) {
            ms = s < live ? ld_dev(p + s * (D + 2) + D) : -INFINITY;
            ls = s < live ? ld_dev(p + s * (D + 2) + D + 1) : 0.0f;
        }
        const float c = (!(ls > 0.0f) && ls == ls) ? 0.0f : expf(ms - M);
        L = fmaf(ls, c, L);
        const int cnt = min(kWave, live - s0);
        for (int j0 = 0; j0 < cnt; j0 += kBatch) {
            if (s0 + j0 > 0) {  // chunks past the first batch
#pragma unroll
                for (int j = 0; j < kBatch; j++)
#pragma unroll
                    for (int i = 0; i < D / kWave; i++)
                        v[j][i] = ld_dev(p + clampc(s0 + j0 + j) * (D + 2) + lane + i * kWave);
            }
#pragma unroll
            for (int j = 0; j < kBatch; j++) {
                // past the last chunk: weight 0 and value 0 (not the re-read
                // chunk's value, which could be infinite)
                const bool on = j0 + j < cnt;
                const float cj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), j0 + j));
#pragma unroll
                for (int i = 0; i < D / kWave; i++) o[i] = fmaf(on ? v[j][i] : 0.0f, on ? cj : 0.0f, o[i]);
            }
        }
    }
    L = wave_sum_rows(L);
    const float inv = L == 0.0f ? 0.0f : 1.0f / L;   // no live position: zeros (cpu_ops.cpp:177-180)
#pragma unroll
    for (int i = 0; i < D / kWave; i++) put_out(a, b, h * D + lane + i * kWave, o[i] * inv);
}

// head-row element held in slot i of lane slice ds
template <int D>
__device__ __forceinline__ int elem_of(int ds, int i) { return (i < 4 ? 0 : D / 2 - 4) + 4 * ds + i; }

template <int D, int GM, bool FINAL, int QK = -1, int MC = kMaxChunk>   // MC: chunk positions whose scores fit in LDS
__global__ __launch_bounds__(kAttnThreads) void gqa_decode_kernel(AttnArgs a) {
    static_assert(QK < 0 || D == 128, "the fused q/k norm + RoPE is for 128-wide heads");
    constexpr int LP = D / 8;                  // lanes per position
    constexpr int PPW = kWave / LP;            // positions per wave per round
    constexpr int PPB = PPW * kAttnWaves;      // positions per workgroup per round
    constexpr int U = 2;                       // rounds per batch of loads (two batches in flight)
    constexpr int STEP = U * PPB;              // positions per batch
    __shared__ float sc[GM][MC];               // scores, then weights
    __shared__ float red[kAttnWaves][GM][D];   // per-wave partial outputs
    __shared__ float hm[GM], hl[GM];

    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    const int kvh = blockIdx.x, split = blockIdx.z;
    const long b = blockIdx.y;
    const int qpos = QK >= 0 ? a.pos[b] : 0;   // read beside the ring state
    int start, len;
    ring_state(a, b, start, len);
    // In a split launch a ring that is short (len <= a.whole, at most one
    // chunk's worth of LDS) is done by chunk 0 alone, which then writes the
    // normalised output itself, with no partials and no count.  The ring
    // lengths live on the device, so this is decided per sequence here.
    const bool whole = !FINAL && len <= a.whole;
    if (whole && split > 0) return;
    const bool fin = FINAL || whole;
    const int t0 = split * a.chunk;
    const int n = whole ? len : min(t0 + a.chunk, len) - t0;     // positions of this chunk
    if (!fin && n <= 0) return;   // past the ring: neither partials nor a count
    const int ps = wid * PPW + lane / LP;          // position slot within a round
    const int ds = lane % LP;                      // this lane's 8-float slice
    const int row = a.nkv * D;                     // cap * row < 2^31 (checked on the host)
    const long off = b * a.seq_stride + (long)kvh * D + 4 * ds;
    const float* kbase = a.kc + off;
    const float* vbase = a.vc + off;
    const int gc = a.gcount;

    // A batch is U rounds of PPB positions.  Batches are double-buffered in
    // registers: the next batch's loads are in flight while this one is
    // used.  Positions past the chunk re-read its last row (n >= 1 inside
    // the loops) and are discarded.
    // QK: the newest row (position len-1) is made here, in this lane's slice
    // layout, by the workgroup whose chunk holds it, substituted for what the
    // caches held at its slot, and written to the caches once made.  The
    // RoPE angles, gammas, raw k and v, the q heads and the first K batch are
    // all loaded before any of them is used, so the loads overlap.
    float knew[8], vnew[8], kr[8];
    float4 rc, rs, gql, gqh, gkl, gkh;   // cos/sin of this lane's four angles; q and k gammas
    const int tnew = QK >= 0 ? len - 1 - t0 : -1;   // its position in this chunk
    const bool owns = QK >= 0 && tnew >= 0 && tnew < n;
    // The loads are unconditional (a branch around a load makes the wave
    // wait for it at the branch's end): a table row (the clamped position's;
    // replaced below when the position is past the table), both gammas (non-
    // null, checked on the host), and the raw k and v of every workgroup.
    const int rpos = QK >= 0 ? min(max(qpos, 0), a.tab_len - 1) : 0;   // tab_len >= 1
    if constexpr (QK >= 0) {
        constexpr int WT = QK < 0 ? ANELM_F32 : QK;
        rc = *reinterpret_cast<const float4*>(a.cos_tab + (long)rpos * 64 + 4 * ds);
        rs = *reinterpret_cast<const float4*>(a.sin_tab + (long)rpos * 64 + 4 * ds);
        gql = load_w4<WT>(a.wq, 4 * ds);
        gqh = load_w4<WT>(a.wq, 4 * ds + 64);
        gkl = load_w4<WT>(a.wk, 4 * ds);
        gkh = load_w4<WT>(a.wk, 4 * ds + 64);
        load8<D, false>(kr, a.kraw + b * a.k_ld + (long)kvh * D + 4 * ds);
        load8<D, false>(vnew, a.vraw + b * a.v_ld + (long)kvh * D + 4 * ds);
    }
    auto load_batch = [&](float (&buf)[U][8], const float* base, int r0) {
#pragma unroll
        for (int u = 0; u < U; u++) load8<D, true>(buf[u], base + ring_slot(a, start, t0, r0 + u * PPB + ps, n) * row);
    };
    // the newest row in place of the slot's old contents (K: knew, V: vnew)
    auto fix_batch = [&](float (&buf)[U][8], const float (&nw)[8], int r0) {
        if constexpr (QK >= 0) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const bool hit = owns && r0 + u * PPB + ps == tnew;
#pragma unroll
                for (int i = 0; i < 8; i++) buf[u][i] = hit ? nw[i] : buf[u][i];
            }
        }
    };

    // phase 1: scores
    {
        float qv[GM][8];
#pragma unroll
        for (int g = 0; g < GM; g++) {
            if constexpr (QK >= 0) {   // branch-free: heads past gc re-read the last one, then zeroed
                const int gg = g < gc ? g : gc - 1;
                load8<D, false>(qv[g], a.q + b * a.q_ld + (long)(kvh * a.groups + a.g0 + gg) * a.q_hs + 4 * ds);
            } else if (g < gc) {
                load8<D, false>(qv[g], a.q + b * a.q_ld + (long)(kvh * a.groups + a.g0 + g) * a.q_hs + 4 * ds);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) qv[g][i] = 0.0f;
            }
        }
        float ka[U][8], kb[U][8];
        if (n > 0) load_batch(ka, kbase, 0);
        if constexpr (QK >= 0) {
            if (qpos != rpos) {   // past the table (uniform): the angles themselves
                float4 fc, fs;
                rope_cs4(qpos, 4 * ds, nullptr, nullptr, 0, a.inv, fc, fs);
                rc = fc;
                rs = fs;
            }
            // the q heads' norm + RoPE, every lane of each 16-lane group
#pragma unroll
            for (int g = 0; g < GM; g++) {
                float4 ol, oh;
                norm_rope128_w(make_float4(qv[g][0], qv[g][1], qv[g][2], qv[g][3]),
                               make_float4(qv[g][4], qv[g][5], qv[g][6], qv[g][7]), true, gql, gqh, rc, rs, a.eps,
                               ol, oh);
                if (g >= gc) ol = oh = make_float4(0.f, 0.f, 0.f, 0.f);   // heads past gc
                qv[g][0] = ol.x; qv[g][1] = ol.y; qv[g][2] = ol.z; qv[g][3] = ol.w;
                qv[g][4] = oh.x; qv[g][5] = oh.y; qv[g][6] = oh.z; qv[g][7] = oh.w;
            }
            if (owns) {   // uniform across the workgroup
                float4 ol, oh;
                norm_rope128_w(make_float4(kr[0], kr[1], kr[2], kr[3]), make_float4(kr[4], kr[5], kr[6], kr[7]), true,
                               gkl, gkh, rc, rs, a.eps, ol, oh);
                knew[0] = ol.x; knew[1] = ol.y; knew[2] = ol.z; knew[3] = ol.w;
                knew[4] = oh.x; knew[5] = oh.y; knew[6] = oh.z; knew[7] = oh.w;
                // The new row goes to the caches now, not behind the
                // outputs: this workgroup's own loads of its slot (the only
                // ones) are replaced by these registers whatever they return.
                if (tid < LP) {   // one 16-lane group stores the row
                    const long slot = ring_slot(a, start, t0, tnew, n);
                    float* kd = const_cast<float*>(kbase) + slot * row;
                    float* vd = const_cast<float*>(vbase) + slot * row;
                    *reinterpret_cast<float4*>(kd) = ol;
                    *reinterpret_cast<float4*>(kd + D / 2) = oh;
                    *reinterpret_cast<float4*>(vd) = make_float4(vnew[0], vnew[1], vnew[2], vnew[3]);
                    *reinterpret_cast<float4*>(vd + D / 2) = make_float4(vnew[4], vnew[5], vnew[6], vnew[7]);
                }
            }
        }
        auto scores = [&](const float (&kx)[U][8], int r0) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int t = r0 + u * PPB + ps;
                float mine = 0.0f;
#pragma unroll
                for (int g = 0; g < GM; g++) {
                    float d = qv[g][0] * kx[u][0];
#pragma unroll
                    for (int i = 1; i < 8; i++) d = fmaf(qv[g][i], kx[u][i], d);
                    d = lp_sum<LP>(d);
                    if (g == ds) mine = d;
                }
                if (t < n && ds < gc) sc[ds][t] = mine * a.scale;
            }
        };
        for (int r0 = 0; r0 < n; r0 += 2 * STEP) {
            if (r0 + STEP < n) load_batch(kb, kbase, r0 + STEP);
            fix_batch(ka, knew, r0);
            scores(ka, r0);
            if (r0 + STEP >= n) break;
            if (r0 + 2 * STEP < n) load_batch(ka, kbase, r0 + 2 * STEP);
            fix_batch(kb, knew, r0 + STEP);
            scores(kb, r0 + STEP);
        }
    }
    // the first V batch is in flight across the softmax
    float va[U][8], vb[U][8];
    if (n > 0) load_batch(va, vbase, 0);
    __syncthreads();

    // phase 2: softmax numerators per head over the chunk
    for (int g = wid; g < gc; g += kAttnWaves) {
        float m = -INFINITY;
        for (int i = lane; i < n; i += kWave) m = fmaxf(m, sc[g][i]);
        m = wave_max_rows(m);
        float l = 0.0f;
        for (int i = lane; i < n; i += kWave) {
            const float e = expf(sc[g][i] - m);
            sc[g][i] = e;
            l += e;
        }
        l = wave_sum_rows(l);
        if (fin) {  // the reference's p = e * (1/sum) (core/cpu_ops.cpp:97-98)
            const float inv = 1.0f / l;
            for (int i = lane; i < n; i += kWave) sc[g][i] = sc[g][i] * inv;
        }
        if (lane == 0) {
            hm[g] = m;
            hl[g] = l;
        }
    }
    __syncthreads();

    // phase 3: weighted sum of V rows
    float acc[GM][8];
#pragma unroll
    for (int g = 0; g < GM; g++)
#pragma unroll
        for (int i = 0; i < 8; i++) acc[g][i] = 0.0f;
    auto accumulate = [&](const float (&vx)[U][8], int r0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = r0 + u * PPB + ps;
            if (t < n) {
#pragma unroll
                for (int g = 0; g < GM; g++) {
                    if (g < gc) {
                        const float w = sc[g][t];
#pragma unroll
                        for (int i = 0; i < 8; i++) acc[g][i] = fmaf(w, vx[u][i], acc[g][i]);
                    }
                }
            }
        }
    };
    for (int r0 = 0; r0 < n; r0 += 2 * STEP) {
        if (r0 + STEP < n) load_batch(vb, vbase, r0 + STEP);
        fix_batch(va, vnew, r0);
        accumulate(va, r0);
        if (r0 + STEP >= n) break;
        if (r0 + 2 * STEP < n) load_batch(va, vbase, r0 + 2 * STEP);
        fix_batch(vb, vnew, r0 + STEP);
        accumulate(vb, r0 + STEP);
    }
    // reduce over the position slots of the wave (lanes with the same slice)
#pragma unroll
    for (int g = 0; g < GM; g++)
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int o = LP; o < kWave; o <<= 1) acc[g][i] += __shfl_xor(acc[g][i], o);
    if (lane < LP) {
#pragma unroll
        for (int g = 0; g < GM; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) red[wid][g][elem_of<D>(ds, i)] = acc[g][i];
    }
    __syncthreads();
    for (int j = tid; j < gc * D; j += kAttnThreads) {
        const int g = j / D, d = j % D;
        float s = red[0][g][d];
#pragma unroll
        for (int w = 1; w < kAttnWaves; w++) s += red[w][g][d];
        const int h = kvh * a.groups + a.g0 + g;
        if (fin) {
            put_out(a, b, h * D + d, s);
        } else {   // device-scope stores: written through for the merging chunk, on any XCD
            float* p = a.ws + ((b * a.nh + h) * a.nsplit + split) * (long)(D + 2);
            st_dev(p + d, s);
            if (d == 0) {
                st_dev(p + D, hm[g]);
                st_dev(p + D + 1, hl[g]);
            }
        }
    }
    if (!fin) {
        // Once every thread's partial stores are acknowledged (the wait
        // covers them), one count per chunk on the (sequence, kv head)
        // counter; the chunk that brings it to the number of live chunks
        // merges, and resets the counter for the next launch.  No fence: the
        // partials were written and are read with device-scope accesses,
        // which bypass the non-coherent per-XCD L2 (a device-scope fence
        // here would write back the whole L2).
        // A bounded launch can hold fewer chunks than a ring longer than its
        // bound needs: then the nsplit launched chunks are the live ones.
        __shared__ int s_last;
        const int live = min((len + a.chunk - 1) / a.chunk, a.nsplit);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            unsigned* c = a.ctr + b * a.nkv + kvh;
            const unsigned prior = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prior == (unsigned)(live - 1);
            if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;
        for (int g = wid; g < gc; g += kAttnWaves) merge_head<D>(a, b, kvh * a.groups + a.g0 + g, lane, live);
    }
}

// Ring append: one workgroup per sequence.
__global__ __launch_bounds__(256) void kv_append_kernel(float* kc, float* vc, int32_t* rs, int32_t* rl,
                                                        const float* k, const float* v, long k_ld, long v_ld,
                                                        int row, int cap, long seq_stride, int vec) {
    __shared__ int s_slot;
    const long b = blockIdx.x;
    if (threadIdx.x == 0) s_slot = ring_advance(rs + b, rl + b, cap);   // qwen3.cpp:475-484
    __syncthreads();
    float* kd = kc + b * seq_stride + (long)s_slot * row;
    float* vd = vc + b * seq_stride + (long)s_slot * row;
    const float* ks = k + b * k_ld;
    const float* vs = v + b * v_ld;
    if (vec) {
        for (int i = threadIdx.x; i < row / 4; i += blockDim.x) {
            reinterpret_cast<float4*>(kd)[i] = reinterpret_cast<const float4*>(ks)[i];
            reinterpret_cast<float4*>(vd)[i] = reinterpret_cast<const float4*>(vs)[i];
        }
    } else {
        for (int i = threadIdx.x; i < row; i += blockDim.x) {
            kd[i] = ks[i];
            vd[i] = vs[i];
        }
    }
}

// Rings [g][b] (g < groups, b < batch, ring g*group_stride + b) each take one
// row: the state update of the append (qwen3.cpp:475-484) without the copy.
__global__ __launch_bounds__(256) void kv_ring_advance_kernel(int32_t* rs, int32_t* rl, long batch, long n,
                                                              long group_stride, int cap) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const long g = i / batch;
    const long r = g * group_stride + (i - g * batch);
    ring_advance(rs + r, rl + r, cap);
}

// Positions per workgroup for a ring of `bound` positions and `pairs`
// (sequence, kv head) pairs: the largest chunk that still gives about
// kTargetBlocks workgroups, at least kMinChunk.
int pick_chunk(long pairs, int bound) {
    for (int c = kMaxChunk; c > kMinChunk; c >>= 1) {
        if (pairs * ((bound + c - 1) / c) >= kTargetBlocks) return c;
    }
    return kMinChunk;
}

int group_max(int D) { return kMaxGD / D < 8 ? kMaxGD / D : 8; }

template <int D, int GM, int QK>
void launch_gm(const AttnArgs& a, long batch, hipStream_t st) {
    if constexpr (GM <= 4) {   // the whole ring's scores within 32 KB of LDS
        if (a.whole_ring) {
            AttnArgs w = a;
            w.nsplit = 1;
            w.chunk = w.whole = a.cap;
            hipLaunchKernelGGL((gqa_decode_kernel<D, GM, true, QK, kWholeRingMax>), dim3(a.nkv, batch, 1),
                               dim3(kAttnThreads), 0, st, w);
            return;
        }
    }
    const dim3 grid(a.nkv, batch, a.nsplit);
    if (a.nsplit == 1) {
        hipLaunchKernelGGL((gqa_decode_kernel<D, GM, true, QK>), grid, dim3(kAttnThreads), 0, st, a);
    } else {
        hipLaunchKernelGGL((gqa_decode_kernel<D, GM, false, QK>), grid, dim3(kAttnThreads), 0, st, a);
    }
}

// One launch per slice of at most group_max(D) q heads of each kv head.  A
// QK launch writes the newest cache row in every slice's launch (the same
// bits each time) and uses it from registers, so no launch depends on the
// order of the others.
template <int D, int QK = -1>
void launch_d(AttnArgs a, long batch, hipStream_t st) {
    const int gmax = group_max(D);
    for (int g0 = 0; g0 < a.groups; g0 += gmax) {
        a.g0 = g0;
        a.gcount = a.groups - g0 < gmax ? a.groups - g0 : gmax;
        if (a.gcount <= 1) launch_gm<D, 1, QK>(a, batch, st);
        else if (a.gcount <= 2) launch_gm<D, 2, QK>(a, batch, st);
        else if (a.gcount <= 4) launch_gm<D, 4, QK>(a, batch, st);
        else launch_gm<D, (kMaxGD / D < 8 ? kMaxGD / D : 8), QK>(a, batch, st);
    }
}

// Split launches: the partials from the workspace's start, and one counter
// per (sequence, kv head) in a region whose place depends on the workspace's
// size alone: its last 64th, from a 256-byte boundary.  Every call given the
// same workspace and size therefore finds each counter at the same address,
// left at zero by the calls before, whatever its batch, chunking or ring
// lengths, and no call's partials reach into the region (checked per call).
size_t partial_bytes(long batch, int nh, int nsplit, int D) {
    return ((size_t)batch * nh * nsplit * (D + 2) * sizeof(float) + 255) & ~(size_t)255;
}
size_t ctr_offset(size_t ws_bytes) { return (ws_bytes - ws_bytes / 64) & ~(size_t)255; }
size_t ctr_slots(size_t ws_bytes) { return (ws_bytes - ctr_offset(ws_bytes)) / sizeof(unsigned); }

// A size that serves every call with at most `batch` sequences and a ring
// bound of at most `cap`.  The chunk follows the batch (pick_chunk), so a
// smaller batch can need more partials than the largest one: the maximum is
// taken over the batches up to `batch`.  Past the batch at which the chunk
// reaches its maximum the partials only grow with the batch, so the loop
// stops there and `batch` itself is counted last.
size_t ws_bytes_for(long batch, int nh, int nkv, int D, int cap) {
    size_t P = 0;
    auto count = [&](long b) {
        const int chunk = pick_chunk(b * nkv, cap);
        const long nsplit = (cap + chunk - 1) / chunk;
        if (nsplit > 1) {
            const size_t pb = partial_bytes(b, nh, (int)nsplit, D);
            P = pb > P ? pb : P;
        }
    };
    for (long b = 1; b < batch && pick_chunk(b * nkv, cap) < kMaxChunk; b++) count(b);
    count(batch);
    if (P == 0) return 0;
    const size_t pairs = (size_t)batch * nkv;
    size_t S = (((P + 256) * 64 / 63 + 256) + 255) & ~(size_t)255;
    if (S < 256 * pairs) S = 256 * pairs;
    while (ctr_offset(S) < P || ctr_slots(S) < pairs) S += 256;
    return S;
}

int check_common(const void* out, const void* q, const void* kc, const void* vc, long batch, int nh, int nkv,
                 int D, long q_ld, int q_hs, long out_ld, int cap, long seq_stride) {
    if (!out || !q || !kc || !vc) return fail(ANELM_ERR_INVALID, "gqa_attention: null pointer");
    if (batch < 0 || nh <= 0 || nkv <= 0 || cap <= 0) return fail(ANELM_ERR_INVALID, "gqa_attention: bad sizes");
    if (batch > 65535 || nkv > 65535) return fail(ANELM_ERR_INVALID, "gqa_attention: batch and n_kv_heads <= 65535");
    if (cap > kMaxSplit * kMinChunk) return fail(ANELM_ERR_INVALID, "gqa_attention: capacity above %d", kMaxSplit * kMinChunk);
    if ((long)cap * nkv * D >= (1L << 31)) return fail(ANELM_ERR_INVALID, "gqa_attention: one sequence's cache above 2^31 floats");
    if (nh % nkv != 0) return fail(ANELM_ERR_INVALID, "gqa_attention: n_heads %d not a multiple of n_kv_heads %d", nh, nkv);
    if (D != 64 && D != 128 && D != 256) return fail(ANELM_ERR_INVALID, "gqa_attention: head_dim %d (64, 128 or 256)", D);
    if (q_hs < D || (batch > 1 && (q_ld < (long)(nh - 1) * q_hs + D || out_ld < (long)nh * D)))
        return fail(ANELM_ERR_INVALID, "gqa_attention: q/out strides overlap");
    if (batch > 1 && seq_stride < (long)cap * nkv * D)
        return fail(ANELM_ERR_INVALID, "gqa_attention: cache_seq_stride smaller than one sequence's cache");
    if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || (q_ld & 3) || (q_hs & 3) || (seq_stride & 3))
        return fail(ANELM_ERR_INVALID, "gqa_attention: q and caches need 16-byte alignment and strides of 4");
    return ANELM_OK;
}

// The chunking of a launch and the workspace it needs, checked before
// anything is launched.
int plan(AttnArgs& a, long batch, int D, int bound, void* ws, size_t ws_bytes) {
    a.groups = a.nh / a.nkv;
    a.scale = 1.0f / sqrtf((float)D);   // core/cpu_ops.cpp:183
    a.chunk = pick_chunk(batch * a.nkv, a.cap);  // from the capacity, so the workspace size holds for any bound
    a.nsplit = (bound + a.chunk - 1) / a.chunk;
    if (a.nsplit < 1) a.nsplit = 1;
    a.whole = a.chunk > kWholeRows ? a.chunk : kWholeRows;   // <= kMaxChunk, the LDS score rows
    if (a.nsplit > 1) {
        const size_t pb = partial_bytes(batch, a.nh, a.nsplit, D);
        if (!ws || pb > ctr_offset(ws_bytes) || (size_t)batch * a.nkv > ctr_slots(ws_bytes))
            return fail(ANELM_ERR_WORKSPACE,
                        "gqa_attention: workspace of %zu bytes too small for %zu bytes of partials and %ld counters",
                        ws_bytes, pb, batch * a.nkv);
        if (!aligned16(ws)) return fail(ANELM_ERR_INVALID, "gqa_attention: workspace not 16-byte aligned");
        a.ctr = reinterpret_cast<unsigned*>(static_cast<char*>(ws) + ctr_offset(ws_bytes));
    }
    a.ws = static_cast<float*>(ws);
    // every ring attended whole (not a bounded launch shorter than the rings)
    a.whole_ring = bound >= a.cap && a.cap <= kWholeRingMax && batch * a.nkv >= kWholeRingPairs;
    return ANELM_OK;
}

// qk: -1, or the weight dtype of a QK launch (head_dim 128)
void dispatch(const AttnArgs& a, long batch, int D, hipStream_t st, int qk = -1) {
    if (qk == ANELM_F32) launch_d<128, ANELM_F32>(a, batch, st);
    else if (qk == ANELM_F16) launch_d<128, ANELM_F16>(a, batch, st);
    else if (qk == ANELM_BF16) launch_d<128, ANELM_BF16>(a, batch, st);
    else if (D == 64) launch_d<64>(a, batch, st);
    else if (D == 128) launch_d<128>(a, batch, st);
    else launch_d<256>(a, batch, st);
}

int run(AttnArgs a, long batch, int D, int bound, void* ws, size_t ws_bytes, hipStream_t st, int qk = -1) {
    const int rc = plan(a, batch, D, bound, ws, ws_bytes);
    if (rc) return rc;
    if (batch == 0) return ANELM_OK;
    dispatch(a, batch, D, st, qk);
    return launch_status("gqa_attention");
}

// The arguments of a QK launch (anelm_gqa_attention_qk), checked.
int qk_args(AttnArgs& a, const char* fn, void* out, int out_f16, const float* q, const float* k, const float* v,
            long q_ld, long k_ld, long v_ld, const void* wq, const void* wk, int w_dtype, const int32_t* pos,
            const float* cos_tab, const float* sin_tab, int tab_len, float theta, float eps, float* k_cache,
            float* v_cache, const int32_t* ring_start, const int32_t* ring_len, long batch, int n_heads,
            int n_kv_heads, long out_ld, int capacity, long cache_seq_stride) {
    int rc = check_common(out, q, k_cache, v_cache, batch, n_heads, n_kv_heads, 128, q_ld, 128, out_ld, capacity,
                          cache_seq_stride);
    if (rc) return rc;
    if (!ring_start || !ring_len || !k || !v || !pos) return fail(ANELM_ERR_INVALID, "%s: null pointer", fn);
    const long row = (long)n_kv_heads * 128;
    if (batch > 1 && (k_ld < row || v_ld < row)) return fail(ANELM_ERR_INVALID, "%s: k/v strides overlap", fn);
    if (tab_len < 1 || !cos_tab || !sin_tab) return fail(ANELM_ERR_INVALID, "%s: needs a RoPE table of >= 1 row", fn);
    if (!wq || !wk) return fail(ANELM_ERR_INVALID, "%s: needs both q and k gammas", fn);
    if (w_dtype < ANELM_F32 || w_dtype > ANELM_BF16) return fail(ANELM_ERR_INVALID, "%s: dtype", fn);
    const bool wal = w_dtype == ANELM_F32 ? aligned16(wq) && aligned16(wk) : aligned8(wq) && aligned8(wk);
    if (!aligned16(k) || !aligned16(v) || ((k_ld | v_ld) & 3) || !wal || !aligned16(cos_tab) || !aligned16(sin_tab))
        return fail(ANELM_ERR_INVALID, "%s: needs 16-byte aligned rows (strides multiples of 4)", fn);
    if (out_f16 < 0 || out_f16 > 2) return fail(ANELM_ERR_INVALID, "%s: out_f16 %d (0, 1 or 2)", fn, out_f16);
    if (out_f16 == 2 && !aligned16(out)) return fail(ANELM_ERR_INVALID, "%s: the tiled output needs 16-byte alignment", fn);
    InvFreq inv;
    rope_inv_freq(&inv, 128, theta);
    if (out_f16) a.out16 = static_cast<uint16_t*>(out);
    else a.out = static_cast<float*>(out);
    if (out_f16 == 2) a.out_cols = n_heads * 128;
    a.q = q; a.kc = k_cache; a.vc = v_cache;
    a.ring_start = ring_start; a.ring_len = ring_len;
    a.nh = n_heads; a.nkv = n_kv_heads;
    a.q_ld = q_ld; a.q_hs = 128; a.out_ld = out_ld;
    a.cap = capacity; a.seq_stride = cache_seq_stride;
    a.kraw = k; a.vraw = v; a.k_ld = k_ld; a.v_ld = v_ld;
    a.wq = wq; a.wk = wk; a.pos = pos;
    a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.tab_len = tab_len; a.eps = eps;
    for (int j = 0; j < 64; j++) a.inv[j] = inv.v[j];
    return ANELM_OK;
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" size_t anelm_gqa_workspace_size(long batch, int n_heads, int n_kv_heads, int head_dim, int capacity) {
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || capacity <= 0) return 0;
    return ws_bytes_for(batch, n_heads, n_kv_heads, head_dim, capacity);
}

extern "C" int anelm_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                                   const int32_t* ring_start, const int32_t* ring_len, long batch, int n_heads,
                                   int n_kv_heads, int head_dim, long q_ld, int q_head_stride, long out_ld,
                                   int capacity, long cache_seq_stride, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    clear_error();
    int rc = check_common(out, q, k_cache, v_cache, batch, n_heads, n_kv_heads, head_dim, q_ld, q_head_stride,
                          out_ld, capacity, cache_seq_stride);
    if (rc) return rc;
    if (!ring_start || !ring_len) return fail(ANELM_ERR_INVALID, "gqa_attention: null ring state");
    AttnArgs a{};
    a.out = out; a.q = q; a.kc = k_cache; a.vc = v_cache;
    a.ring_start = ring_start; a.ring_len = ring_len;
    a.nh = n_heads; a.nkv = n_kv_heads;
    a.q_ld = q_ld; a.q_hs = q_head_stride; a.out_ld = out_ld;
    a.cap = capacity; a.seq_stride = cache_seq_stride;
    return run(a, batch, head_dim, capacity, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int anelm_gqa_attention_f16(uint16_t* out16, const float* q, const float* k_cache, const float* v_cache,
                                       const int32_t* ring_start, const int32_t* ring_len, long batch, int n_heads,
                                       int n_kv_heads, int head_dim, long q_ld, int q_head_stride, long out_ld,
                                       int capacity, long cache_seq_stride, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    clear_error();
    int rc = check_common(out16, q, k_cache, v_cache, batch, n_heads, n_kv_heads, head_dim, q_ld, q_head_stride,
                          out_ld, capacity, cache_seq_stride);
    if (rc) return rc;
    if (!ring_start || !ring_len) return fail(ANELM_ERR_INVALID, "gqa_attention: null ring state");
    AttnArgs a{};
    a.out16 = out16; a.q = q; a.kc = k_cache; a.vc = v_cache;
    a.ring_start = ring_start; a.ring_len = ring_len;
    a.nh = n_heads; a.nkv = n_kv_heads;
    a.q_ld = q_ld; a.q_hs = q_head_stride; a.out_ld = out_ld;
    a.cap = capacity; a.seq_stride = cache_seq_stride;
    return run(a, batch, head_dim, capacity, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int anelm_gqa_attention_bounded(float* out, const float* q, const float* k_cache, const float* v_cache,
                                           const int32_t* ring_start, const int32_t* ring_len, long batch,
                                           int n_heads, int n_kv_heads, int head_dim, long q_ld, int q_head_stride,
                                           long out_ld, int capacity, long cache_seq_stride, int len_bound,
                                           void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_common(out, q, k_cache, v_cache, batch, n_heads, n_kv_heads, head_dim, q_ld, q_head_stride,
                          out_ld, capacity, cache_seq_stride);
    if (rc) return rc;
    if (!ring_start || !ring_len) return fail(ANELM_ERR_INVALID, "gqa_attention: null ring state");
    if (len_bound <= 0) return fail(ANELM_ERR_INVALID, "gqa_attention: len_bound %d", len_bound);
    AttnArgs a{};
    a.out = out; a.q = q; a.kc = k_cache; a.vc = v_cache;
    a.ring_start = ring_start; a.ring_len = ring_len;
    a.nh = n_heads; a.nkv = n_kv_heads;
    a.q_ld = q_ld; a.q_hs = q_head_stride; a.out_ld = out_ld;
    a.cap = capacity; a.seq_stride = cache_seq_stride;
    return run(a, batch, head_dim, len_bound < capacity ? len_bound : capacity, workspace, workspace_bytes,
               as_stream(stream));
}

extern "C" int anelm_gqa_attention_ring(float* out, const float* q, const float* k_cache, const float* v_cache,
                                        int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                                        int cache_start, int cache_len, int cache_capacity, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_common(out, q, k_cache, v_cache, 1, n_heads, n_kv_heads, head_dim, 0, q_head_stride, 0,
                          cache_capacity, 0);
    if (rc) return rc;
    if (cache_len > cache_capacity || (cache_len > 0 && (cache_start < 0 || cache_start >= cache_capacity)))
        return fail(ANELM_ERR_RANGE, "gqa_attention: ring start %d / len %d outside capacity %d", cache_start,
                    cache_len, cache_capacity);
    AttnArgs a{};
    a.out = out; a.q = q; a.kc = k_cache; a.vc = v_cache;
    a.start0 = cache_len > 0 ? cache_start : 0;
    a.len0 = cache_len > 0 ? cache_len : 0;
    a.nh = n_heads; a.nkv = n_kv_heads;
    a.q_hs = q_head_stride; a.out_ld = (long)n_heads * head_dim;
    a.cap = cache_capacity; a.seq_stride = (long)cache_capacity * n_kv_heads * head_dim;
    return run(a, 1, head_dim, a.len0 > 0 ? a.len0 : 1, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int anelm_kv_ring_append(float* k_cache, float* v_cache, int32_t* ring_start, int32_t* ring_len,
                                    const float* k, const float* v, long k_ld, long v_ld, long batch,
                                    int n_kv_heads, int head_dim, int capacity, long cache_seq_stride,
                                    void* stream) {
    clear_error();
    if (!k_cache || !v_cache || !ring_start || !ring_len || !k || !v)
        return fail(ANELM_ERR_INVALID, "kv_ring_append: null pointer");
    if (batch < 0 || n_kv_heads <= 0 || head_dim <= 0 || capacity <= 0)
        return fail(ANELM_ERR_INVALID, "kv_ring_append: bad sizes");
    const long row = (long)n_kv_heads * head_dim;
    if (row > (1L << 30)) return fail(ANELM_ERR_INVALID, "kv_ring_append: row too long");
    if (batch > 1 && (cache_seq_stride < (long)capacity * row || k_ld < row || v_ld < row))
        return fail(ANELM_ERR_INVALID, "kv_ring_append: strides overlap");
    if (batch == 0) return ANELM_OK;
    const int vec = aligned16(k_cache) && aligned16(v_cache) && aligned16(k) && aligned16(v) && !(row & 3) &&
                    !(k_ld & 3) && !(v_ld & 3) && !(cache_seq_stride & 3);
    hipLaunchKernelGGL(kv_append_kernel, dim3(batch), dim3(256), 0, as_stream(stream), k_cache, v_cache, ring_start,
                       ring_len, k, v, k_ld, v_ld, (int)row, capacity, cache_seq_stride, vec);
    return launch_status("kv_ring_append");
}

extern "C" int anelm_kv_ring_advance(int32_t* ring_start, int32_t* ring_len, long batch, int groups,
                                     long group_stride, int capacity, void* stream) {
    clear_error();
    if (!ring_start || !ring_len) return fail(ANELM_ERR_INVALID, "kv_ring_advance: null pointer");
    if (batch < 0 || groups < 0 || capacity <= 0 || (groups > 1 && group_stride < batch))
        return fail(ANELM_ERR_INVALID, "kv_ring_advance: bad sizes");
    const long n = batch * groups;
    if (n == 0) return ANELM_OK;
    if (n > (1L << 31)) return fail(ANELM_ERR_INVALID, "kv_ring_advance: too many rings");
    hipLaunchKernelGGL(kv_ring_advance_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream),
                       ring_start, ring_len, batch, n, group_stride, capacity);
    return launch_status("kv_ring_advance");
}

extern "C" int anelm_gqa_attention_qk(void* out, int out_f16, const float* q, const float* k, const float* v,
                                      long q_ld, long k_ld, long v_ld, const void* wq, const void* wk, int w_dtype,
                                      const int32_t* pos, const float* cos_tab, const float* sin_tab, int tab_len,
                                      float theta, float eps, float* k_cache, float* v_cache,
                                      const int32_t* ring_start, const int32_t* ring_len, long batch, int n_heads,
                                      int n_kv_heads, long out_ld, int capacity, long cache_seq_stride,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    AttnArgs a{};
    const int rc = qk_args(a, "gqa_attention_qk", out, out_f16, q, k, v, q_ld, k_ld, v_ld, wq, wk, w_dtype, pos,
                           cos_tab, sin_tab, tab_len, theta, eps, k_cache, v_cache, ring_start, ring_len, batch,
                           n_heads, n_kv_heads, out_ld, capacity, cache_seq_stride);
    if (rc) return rc;
    return run(a, batch, 128, capacity, workspace, workspace_bytes, as_stream(stream), w_dtype);
}

// The same with the rings' advance in the call (qwen3.cpp:475-484, then the
// append and attention of :487-492): every argument and the workspace are
// checked before anything is launched, then one launch advances the batch's
// rings and the next makes, stores and attends over the new rows.
extern "C" int anelm_gqa_attention_qk_append(void* out, int out_f16, const float* q, const float* k,
                                             const float* v, long q_ld, long k_ld, long v_ld, const void* wq,
                                             const void* wk, int w_dtype, const int32_t* pos, const float* cos_tab,
                                             const float* sin_tab, int tab_len, float theta, float eps,
                                             float* k_cache, float* v_cache, int32_t* ring_start, int32_t* ring_len,
                                             long batch, int n_heads, int n_kv_heads, long out_ld, int capacity,
                                             long cache_seq_stride, void* workspace, size_t workspace_bytes,
                                             void* stream) {
    clear_error();
    AttnArgs a{};
    int rc = qk_args(a, "gqa_attention_qk_append", out, out_f16, q, k, v, q_ld, k_ld, v_ld, wq, wk, w_dtype, pos,
                     cos_tab, sin_tab, tab_len, theta, eps, k_cache, v_cache, ring_start, ring_len, batch, n_heads,
                     n_kv_heads, out_ld, capacity, cache_seq_stride);
    if (rc) return rc;
    rc = plan(a, batch, 128, capacity, workspace, workspace_bytes);
    if (rc) return rc;
    if (batch == 0) return ANELM_OK;
    const hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(kv_ring_advance_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, st, ring_start,
                       ring_len, batch, batch, batch, capacity);
    dispatch(a, batch, 128, st, w_dtype);
    return launch_status("gqa_attention_qk_append");
}
