// The five layer ops of models/llm/qwen3.cpp:502-528 in one launch, for
// callers that hold all of a layer's op inputs at once (the op chain without
// the contractions between its ops, e.g. decode-shaped chains whose five
// separate launches are each a few microseconds of latency):
//   xn_in   = rmsnorm(x) * w_in                     (:503)
//   q, k    = per-head rmsnorm, then Qwen3 RoPE      (:444-472)
//   x       = x + attn;  xn_post = rmsnorm(x) * w_post   (:516-518)
//   h       = silu(g) * u                           (core/ane_runtime.cpp:393-395)
//   x       = x + mlp                               (:527)
// The three parts share no data, so the grid is three block ranges and no
// block waits for another:
//   - the x chain, one token row per rms_row_geometry lane group (a block,
//     or each wave of a block when the geometry gives one wave per row), with
//     the lane layout of the separate row RMSNorm, so both norms sum their
//     squares in the same order and every output has the separate kernels'
//     bits; x is read once and its final value (x + attn + mlp) written at
//     once; both norms' sums share one LDS exchange and barrier (none for a
//     one-wave row);
//   - the q/k heads, 16 lanes per head (norm_rope128_w, the separate
//     kernel's arithmetic); with nq and nk multiples of 4 each wave takes 4
//     heads of one token, so its position is a scalar load and every load
//     of the wave goes out before the first wait;
//   - the SwiGLU, two float4 of g, u and h per lane.
#include "anelm_common.hpp"

namespace anelm {
namespace {

struct LayerArgs {
    float* x;
    float* xn_in;
    float* xn_post;
    const float* attn;
    const float* mlp;
    float* q;
    float* k;
    float* h;
    const float* g;
    const float* u;
    const void* w_in;
    const void* w_post;
    const void* wq;
    const void* wk;
    const int32_t* pos;
    const float* cos_tab;
    const float* sin_tab;
    int tab_len;
    int H;
    int nq, nk;
    long T;
    long n4;          // float4 of the SwiGLU (T * I / 4)
    int row_threads;  // lanes per token row (rms_row_geometry)
    int rows_per_block;  // blockDim.x / row_threads (> 1 only for one-wave rows)
    int row_blocks;   // [0, row_blocks): x chain
    int qk_blocks;    // then the q/k heads
    float eps;
};

// One token row's x chain; lane layout and reduction order of
// rmsnorm_row_kernel<NV, DT, ...> with a.row_threads lanes.  FULL: every lane
// holds NV float4 of the row (hidden == 4 * NV * row_threads, every Qwen3
// shape), so nothing is guarded; a guarded store let the compiler sink the
// mlp load, its only use, into the guard, behind a wait for the others.
// With several rows per block each row is one wave (no LDS exchange, no
// barrier), and a wave past the last row returns at once.
template <int NV, int DT, bool FULL>
__device__ __forceinline__ void x_chain(const LayerArgs& a, long blk) {
    __shared__ float part[2][16];
    const int nthr = a.row_threads, nw = nthr >> 6;
    const int tid = a.rows_per_block > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
    const long row = blk * a.rows_per_block + (a.rows_per_block > 1 ? (long)(threadIdx.x >> 6) : 0L);
    if (row >= a.T) return;   // a whole wave of the last block (one row per block: blk < T always)
    const int dim = a.H;
    float* xr = a.x + row * dim;
    const float* ar = a.attn + row * dim;
    const float* mr = a.mlp + row * dim;
    int col[NV];
    bool live[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = (i * nthr + tid) * 4;
        live[i] = FULL || c < dim;
        col[i] = live[i] ? c : dim - 4;
    }
    Gamma4<DT> gi[NV], gp[NV];
    float4 v[NV], at[NV], ml[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        gi[i].load(a.w_in, col[i]);
        gp[i].load(a.w_post, col[i]);
        v[i] = *reinterpret_cast<const float4*>(xr + col[i]);
        at[i] = ld_nt(reinterpret_cast<const float4*>(ar + col[i]));
        ml[i] = ld_nt(reinterpret_cast<const float4*>(mr + col[i]));
    }
    // x + attn and the final x + attn + mlp are known now: the final x is
    // stored at once, and both norms' sums of squares (each in
    // rmsnorm_row_kernel's order) share one LDS exchange and one barrier
    float4 v2[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        v2[i].x = v[i].x + at[i].x;   // :516
        v2[i].y = v[i].y + at[i].y;
        v2[i].z = v[i].z + at[i].z;
        v2[i].w = v[i].w + at[i].w;
        float4 v3;
        v3.x = v2[i].x + ml[i].x;     // :527
        v3.y = v2[i].y + ml[i].y;
        v3.z = v2[i].z + ml[i].z;
        v3.w = v2[i].w + ml[i].w;
        if (FULL || live[i]) st_nt(reinterpret_cast<float4*>(xr + col[i]), v3);
    }
    float ss1 = 0.f, ss2 = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const float4 b = FULL || live[i] ? v[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 c = FULL || live[i] ? v2[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        ss1 = fmaf(b.x, b.x, ss1);
        ss1 = fmaf(b.y, b.y, ss1);
        ss1 = fmaf(b.z, b.z, ss1);
        ss1 = fmaf(b.w, b.w, ss1);
        ss2 = fmaf(c.x, c.x, ss2);
        ss2 = fmaf(c.y, c.y, ss2);
        ss2 = fmaf(c.z, c.z, ss2);
        ss2 = fmaf(c.w, c.w, ss2);
    }
    ss1 = wave_sum_rows(ss1);
    ss2 = wave_sum_rows(ss2);
    if (nw > 1) {
        if ((tid & 63) == 0) {
            part[0][tid >> 6] = ss1;
            part[1][tid >> 6] = ss2;
        }
        __syncthreads();
        ss1 = part[0][0];
        ss2 = part[1][0];
        for (int w = 1; w < nw; w++) {
            ss1 += part[0][w];
            ss2 += part[1][w];
        }
    }
    const float s1 = 1.0f / sqrtf(ss1 / (float)dim + a.eps);
    const float s2 = 1.0f / sqrtf(ss2 / (float)dim + a.eps);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        if (FULL || live[i]) {
            const float4 w1 = gi[i].get(), w2 = gp[i].get();
            float4 o1, o2;
            o1.x = (v[i].x * s1) * w1.x;   // :503
            o1.y = (v[i].y * s1) * w1.y;
            o1.z = (v[i].z * s1) * w1.z;
            o1.w = (v[i].w * s1) * w1.w;
            o2.x = (v2[i].x * s2) * w2.x;  // :518
            o2.y = (v2[i].y * s2) * w2.y;
            o2.z = (v2[i].z * s2) * w2.z;
            o2.w = (v2[i].w * s2) * w2.w;
            st_nt(reinterpret_cast<float4*>(a.xn_in + row * dim + col[i]), o1);
            st_nt(reinterpret_cast<float4*>(a.xn_post + row * dim + col[i]), o2);
        }
    }
}

// The q/k part takes one head per 16-lane group, four heads to a wave.
// Against 8 per wave (two per group, as qknorm_rope128_w8_kernel) the heads
// spread over twice the waves and each wave's dependent chain is half as
// long: 4B decode at 64 tokens 5.92 -> 5.23 us per layer, the prefill shapes
// and the 0.6B decode unchanged within run-to-run noise.  (The separate kernel keeps
// 8: at 64 tokens 4 per wave measured 4.29 against 4.07 us there.)  The
// arithmetic per head is the same either way.

// q/k heads: flat index over the T*nq q heads then the T*nk k heads, one
// head per 16-lane group.  W4: each wave owns 4 consecutive heads (all of one
// token, nq and nk multiples of 4), so the token is wave-uniform and its
// position a scalar load; else each group loads its own token's position.
template <int DT, bool W4>
__device__ __forceinline__ void qk_heads(const LayerArgs& a, const InvFreq& inv, int blk) {
    const uint32_t nqh = (uint32_t)a.T * (uint32_t)a.nq;
    const uint32_t heads = nqh + (uint32_t)a.T * (uint32_t)a.nk;
    const int j0 = 4 * (threadIdx.x & 15);
    const uint32_t head = (uint32_t)blk * (blockDim.x >> 4) + (threadIdx.x >> 4);
    if (W4) {
        if ((head & ~3u) >= heads) return;   // whole wave (heads is a multiple of 4)
    } else if (head >= heads) {
        return;   // whole 16-lane group
    }
    const bool isq = head < nqh;
    uint32_t t = isq ? head / (uint32_t)a.nq : (head - nqh) / (uint32_t)a.nk;
    if (W4) t = __builtin_amdgcn_readfirstlane(t);
    const int p = a.pos[t];
    Gamma4<DT> glo, ghi;
    glo.load(isq ? a.wq : a.wk, j0);
    ghi.load(isq ? a.wq : a.wk, j0 + 64);
    float* v = isq ? a.q + (long)t * a.nq * 128 + (long)(head - t * (uint32_t)a.nq) * 128
                   : a.k + (long)t * a.nk * 128 + (long)(head - nqh - t * (uint32_t)a.nk) * 128;
    const float4 lo = ld_nt(reinterpret_cast<const float4*>(v + j0));
    const float4 hi = ld_nt(reinterpret_cast<const float4*>(v + 64 + j0));
    const int pr = p < 0 ? 0 : (p >= a.tab_len ? a.tab_len - 1 : p);
    float4 c = *reinterpret_cast<const float4*>(a.cos_tab + (long)pr * 64 + j0);
    float4 s = *reinterpret_cast<const float4*>(a.sin_tab + (long)pr * 64 + j0);
    if (p != pr) rope_cs4(p, j0, a.cos_tab, a.sin_tab, a.tab_len, inv.v, c, s);   // past the table
    float4 ol, oh;
    norm_rope128_w(lo, hi, true, glo.get(), ghi.get(), c, s, a.eps, ol, oh);
    st_nt(reinterpret_cast<float4*>(v + j0), ol);
    st_nt(reinterpret_cast<float4*>(v + 64 + j0), oh);
}

// two float4 of g, u and h per lane, a block's lanes on consecutive float4
// (one per lane measured slower at 64 and 2048 tokens: 5.92 against 5.24 us
// per layer at 4B decode)
__device__ __forceinline__ void swiglu(const LayerArgs& a, int blk) {
    const long i0 = (long)blk * 2 * blockDim.x + threadIdx.x;
    float4 gv[2], uv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const long i = i0 + (long)j * blockDim.x;
        const long ic = i < a.n4 ? i : a.n4 - 1;   // clamped: loads stay unconditional
        gv[j] = ld_nt(reinterpret_cast<const float4*>(a.g) + ic);
        uv[j] = ld_nt(reinterpret_cast<const float4*>(a.u) + ic);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const long i = i0 + (long)j * blockDim.x;
        float4 r;
        r.x = silu_ref(gv[j].x) * uv[j].x;
        r.y = silu_ref(gv[j].y) * uv[j].y;
        r.z = silu_ref(gv[j].z) * uv[j].z;
        r.w = silu_ref(gv[j].w) * uv[j].w;
        if (i < a.n4) st_nt(reinterpret_cast<float4*>(a.h) + i, r);
    }
}

template <int NV, int DT, bool W4, bool FULL>
__global__ __launch_bounds__(1024) void layer_ops_kernel(LayerArgs a, const InvFreq inv) {
    int blk = blockIdx.x;
    if (blk < a.row_blocks) {
        x_chain<NV, DT, FULL>(a, blk);
        return;
    }
    blk -= a.row_blocks;
    if (blk < a.qk_blocks) {
        qk_heads<DT, W4>(a, inv, blk);
        return;
    }
    swiglu(a, blk - a.qk_blocks);
}

template <int NV, int DT>
void launch_layer(const LayerArgs& a, const InvFreq& inv, bool w4, int threads, int blocks, hipStream_t st) {
    const dim3 grd((unsigned)blocks), blk((unsigned)threads);
    const bool full = a.H == 4 * NV * a.row_threads;
    if (w4 && full) layer_ops_kernel<NV, DT, true, true><<<grd, blk, 0, st>>>(a, inv);
    else if (w4) layer_ops_kernel<NV, DT, true, false><<<grd, blk, 0, st>>>(a, inv);
    else if (full) layer_ops_kernel<NV, DT, false, true><<<grd, blk, 0, st>>>(a, inv);
    else layer_ops_kernel<NV, DT, false, false><<<grd, blk, 0, st>>>(a, inv);
}

template <int DT>
void launch_layer_dt(int nv, const LayerArgs& a, const InvFreq& inv, bool w4, int threads, int blocks,
                     hipStream_t st) {
    switch (nv) {
        case 1: launch_layer<1, DT>(a, inv, w4, threads, blocks, st); break;
        case 2: launch_layer<2, DT>(a, inv, w4, threads, blocks, st); break;
        default: launch_layer<4, DT>(a, inv, w4, threads, blocks, st); break;
    }
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_layer_ops(float* x, float* xn_in, float* xn_post, const float* attn, const float* mlp, float* q,
                               float* k, float* h, const float* g, const float* u, const void* w_in,
                               const void* w_post, const void* wq, const void* wk, int w_dtype, const int32_t* pos,
                               const float* cos_tab, const float* sin_tab, int tab_len, float theta, long T,
                               int hidden, int nq, int nk, long inter, float eps, void* stream) {
    const char* fn = "anelm_layer_ops";
    if (!x || !xn_in || !xn_post || !attn || !mlp || !q || !k || !h || !g || !u || !w_in || !w_post || !wq || !wk ||
        !pos || !cos_tab || !sin_tab)
        return fail(ANELM_ERR_INVALID, "%s: null pointer", fn);
    if (T <= 0 || hidden <= 0 || hidden % 4 || hidden > 16384 || nq <= 0 || nk <= 0 || inter <= 0 || inter % 4 ||
        tab_len <= 0)
        return fail(ANELM_ERR_INVALID, "%s: bad sizes (hidden a multiple of 4 up to 16384, inter a multiple of 4, "
                                       "a RoPE table)", fn);
    if (T * (nq + nk) > 0x7FFFFFFFL || T > 0x7FFFFFFFL || T * inter / 4 > (long)0x7FFFFFFF * 256)
        return fail(ANELM_ERR_INVALID, "%s: too large", fn);
    if (w_dtype < ANELM_F32 || w_dtype > ANELM_BF16) return fail(ANELM_ERR_INVALID, "%s: dtype", fn);
    const bool wal = w_dtype == ANELM_F32 ? aligned16(w_in) && aligned16(w_post) && aligned16(wq) && aligned16(wk)
                                          : aligned8(w_in) && aligned8(w_post) && aligned8(wq) && aligned8(wk);
    if (!aligned16(x) || !aligned16(xn_in) || !aligned16(xn_post) || !aligned16(attn) || !aligned16(mlp) ||
        !aligned16(q) || !aligned16(k) || !aligned16(h) || !aligned16(g) || !aligned16(u) || !wal ||
        !aligned16(cos_tab) || !aligned16(sin_tab))
        return fail(ANELM_ERR_INVALID, "%s: needs 16-byte aligned rows", fn);
    int nv, row_threads;
    rms_row_geometry(T, hidden / 4, nv, row_threads);
    // one-wave rows go four to a 256-lane block (the q/k and SwiGLU blocks
    // take the same block size)
    const int rpb = row_threads == 64 ? 4 : 1;
    const int threads = row_threads * rpb;
    const bool w4 = nq % 4 == 0 && nk % 4 == 0;
    const long heads = T * (nq + nk);
    const long qk_blocks = (heads + threads / 16 - 1) / (threads / 16);   // one head per 16 lanes
    const long n4 = T * inter / 4;
    const long silu_blocks = (n4 + 2L * threads - 1) / (2L * threads);
    const long row_blocks = (T + rpb - 1) / rpb;
    const long blocks = row_blocks + qk_blocks + silu_blocks;
    if (blocks > 0x7FFFFFFFL) return fail(ANELM_ERR_INVALID, "%s: too large", fn);
    LayerArgs a;
    a.x = x;
    a.xn_in = xn_in;
    a.xn_post = xn_post;
    a.attn = attn;
    a.mlp = mlp;
    a.q = q;
    a.k = k;
    a.h = h;
    a.g = g;
    a.u = u;
    a.w_in = w_in;
    a.w_post = w_post;
    a.wq = wq;
    a.wk = wk;
    a.pos = pos;
    a.cos_tab = cos_tab;
    a.sin_tab = sin_tab;
    a.tab_len = tab_len;
    a.H = hidden;
    a.nq = nq;
    a.nk = nk;
    a.T = T;
    a.n4 = n4;
    a.row_threads = row_threads;
    a.rows_per_block = rpb;
    a.row_blocks = (int)row_blocks;
    a.qk_blocks = (int)qk_blocks;
    a.eps = eps;
    InvFreq inv;
    rope_inv_freq(&inv, 128, theta);
    clear_error();
    hipStream_t st = as_stream(stream);
    switch (w_dtype) {
        case ANELM_F32: launch_layer_dt<ANELM_F32>(nv, a, inv, w4, threads, (int)blocks, st); break;
        case ANELM_F16: launch_layer_dt<ANELM_F16>(nv, a, inv, w4, threads, (int)blocks, st); break;
        default: launch_layer_dt<ANELM_BF16>(nv, a, inv, w4, threads, (int)blocks, st); break;
    }
    return launch_status("layer_ops");
}
