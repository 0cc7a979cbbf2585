// RMSNorm, fused residual-add + RMSNorm, per-head q/k RMSNorm + RoPE, the
// apply_rope_cached variant and the RoPE table, for gfx950.
//
// All of these are HBM-bound (< 1 flop/byte): every activation is read
// from HBM once and written once, with 16-byte accesses, and reductions are
// wave shuffles plus at most one LDS exchange of per-wave partials.
#include <algorithm>
#include <cmath>

#include "anelm_common.hpp"

namespace anelm {

// ---------------------------------------------------------------- RMSNorm
// core/cpu_ops.cpp:25-31: ss = sum x^2; s = 1/sqrtf(ss/dim + eps) (true
// divide and square root, correctly rounded); out = (x*s)*w with the two
// products rounded separately.  With ADD, first x += y (qwen3.cpp:516) and
// the updated x is written back.
//
// One workgroup per row, ceil(dim/(4*NV))/64 waves, NV float4 per lane:
// the row is read once into registers (non-temporal: it is not re-read),
// reduced with wave shuffles plus one LDS exchange of the per-wave
// partials, and written once.  Light workgroups (two float4 per lane at
// H=4096) keep many rows in flight per CU, which measured faster than one
// wave per row holding the whole row.  The row is entirely in registers
// before anything is written, so out may alias x and y may alias out.
// With O16 the output is fp16 rounded to nearest even: the activation
// conversion at the ANE kernel inputs (core/ane_runtime.cpp:604-612) applied
// to the RMSNorm's fp32 result, for a projection that takes fp16 inputs.
__device__ __forceinline__ uint32_t f16_bits_rne(float v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, to_f16(v));
}

// Every load is issued unconditionally, from a column clamped into the row
// (lanes past its end load a valid element and discard it): a load inside a
// branch makes the wave wait for it where the branch ends, which serialised
// the gamma loads behind the reduction (one memory round trip each).  The
// gammas are fetched together with the row, as raw bits.
// FULL: the row fills every lane's NV float4 (dim == 4 * NV * blockDim.x,
// every Qwen3 shape), so no lane is guarded.  (Two rows per workgroup, both
// in flight with the gammas loaded once, measured 2 points slower for the
// RMSNorm and 7 for add + RMSNorm at 8192 rows of 4096.)
// TILE (with O16, dim a multiple of 32): the fp16 output in the tiled layout
// of anelm_proj_tile_f16 (rows of 16, steps of 32 columns, each 16 x 32 block
// one contiguous 1 KB piece), the input layout of the tiled projection.
template <int NV, int DT, bool ADD, bool O16 = false, bool FULL = false, bool TILE = false>
__global__ __launch_bounds__(1024) void rmsnorm_row_kernel(void* out, float* x, const float* y,
                                                           const void* w, long rows, int dim,
                                                           long ld_x, long ld_y, long ld_out,
                                                           float eps) {
    __shared__ float part[16];
    const int tid = threadIdx.x, nthr = blockDim.x;
    const long row = blockIdx.x;
    float* xr = x + row * ld_x;
    int col[NV];
    bool live[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = (i * nthr + tid) * 4;
        live[i] = FULL || c < dim;
        col[i] = live[i] ? c : dim - 4;
    }
    Gamma4<DT> g[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) g[i].load(w, col[i]);
    float4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++)
        v[i] = ADD ? *reinterpret_cast<const float4*>(xr + col[i]) : ld_nt(reinterpret_cast<const float4*>(xr + col[i]));
    if (ADD) {
        const float* yr = y + row * ld_y;
        float4 b[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) b[i] = ld_nt(reinterpret_cast<const float4*>(yr + col[i]));
#pragma unroll
        for (int i = 0; i < NV; i++) {
            v[i].x = v[i].x + b[i].x;
            v[i].y = v[i].y + b[i].y;
            v[i].z = v[i].z + b[i].z;
            v[i].w = v[i].w + b[i].w;
            if (FULL || live[i]) *reinterpret_cast<float4*>(xr + col[i]) = v[i];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const float4 a = FULL || live[i] ? v[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        ss = fmaf(a.x, a.x, ss);
        ss = fmaf(a.y, a.y, ss);
        ss = fmaf(a.z, a.z, ss);
        ss = fmaf(a.w, a.w, ss);
    }
    ss = wave_sum_rows(ss);
    const int nw = nthr >> 6;
    if (nw > 1) {
        if ((tid & 63) == 0) part[tid >> 6] = ss;
        __syncthreads();
        ss = part[0];
        for (int k = 1; k < nw; k++) ss += part[k];
    }
    const float s = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        if (FULL || live[i]) {
            const float4 wv = g[i].get();
            const int c = col[i];
            float4 o;
            o.x = (v[i].x * s) * wv.x;
            o.y = (v[i].y * s) * wv.y;
            o.z = (v[i].z * s) * wv.z;
            o.w = (v[i].w * s) * wv.w;
            if constexpr (O16) {
                const uint2 h = make_uint2(f16_bits_rne(o.x) | (f16_bits_rne(o.y) << 16),
                                           f16_bits_rne(o.z) | (f16_bits_rne(o.w) << 16));
                if constexpr (TILE) {
                    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + tiled_index(row, c, dim)) = h;
                } else {
                    uint16_t* orow = static_cast<uint16_t*>(out) + row * ld_out;
                    *reinterpret_cast<uint2*>(orow + c) = h;
                }
            } else {
                st_nt(reinterpret_cast<float4*>(static_cast<float*>(out) + row * ld_out + c), o);
            }
        }
    }
}

// Any dim / alignment: one 256-thread block per row, two passes over the row
// (the second re-reads x, which the same thread wrote in the ADD case).
template <int DT, bool ADD, bool O16 = false>
__global__ __launch_bounds__(256) void rmsnorm_block_kernel(void* out, float* x, const float* y,
                                                            const void* w, long rows, int dim,
                                                            long ld_x, long ld_y, long ld_out,
                                                            float eps) {
    __shared__ float part[4];
    const long row = blockIdx.x;
    float* xr = x + row * ld_x;
    const float* yr = ADD ? y + row * ld_y : nullptr;
    float ss = 0.f;
    for (int c = threadIdx.x; c < dim; c += 256) {
        float a = xr[c];
        if (ADD) {
            a = a + yr[c];
            xr[c] = a;
        }
        ss = fmaf(a, a, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float s = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int c = threadIdx.x; c < dim; c += 256) {
        const float o = (xr[c] * s) * load_w<DT>(w, c);
        if constexpr (O16) static_cast<uint16_t*>(out)[row * ld_out + c] = (uint16_t)f16_bits_rne(o);
        else static_cast<float*>(out)[row * ld_out + c] = o;
    }
}

template <int DT, bool ADD, bool O16 = false, bool TILE = false>
static int launch_rmsnorm_dt(void* out, float* x, const float* y, const void* w, long rows,
                             int dim, long ld_x, long ld_y, long ld_out, float eps,
                             hipStream_t st) {
    const bool vec = (dim % 4 == 0) && (ld_x % 4 == 0) && (ld_out % 4 == 0) && aligned16(x) &&
                     (O16 ? aligned8(out) : aligned16(out)) &&
                     (DT == ANELM_F32 ? aligned16(w) : aligned8(w)) &&
                     (!ADD || ((ld_y % 4 == 0) && aligned16(y)));
    const int nvec = dim / 4;  // float4 per row
    if (TILE && !(vec && nvec <= 1024 * 4))
        return fail(ANELM_ERR_INVALID, "rmsnorm: the tiled output needs 16-byte aligned x, ld_x a multiple of 4, "
                                       "an 8-byte aligned gamma and dim <= 16384");
    if (vec && nvec <= 1024 * 4) {
        int nv, threads;
        rms_row_geometry(rows, nvec, nv, threads);
        const dim3 grd((unsigned)rows);
        const bool full = nvec == nv * threads;
#define ANELM_RMS_ROW(NV_, FULL_) \
    rmsnorm_row_kernel<NV_, DT, ADD, O16, FULL_, TILE><<<grd, threads, 0, st>>>(out, x, y, w, rows, dim, ld_x, ld_y, ld_out, eps)
        if (nv == 1) full ? ANELM_RMS_ROW(1, true) : ANELM_RMS_ROW(1, false);
        else if (nv == 2) full ? ANELM_RMS_ROW(2, true) : ANELM_RMS_ROW(2, false);
        else full ? ANELM_RMS_ROW(4, true) : ANELM_RMS_ROW(4, false);
#undef ANELM_RMS_ROW
        return launch_status("rmsnorm");
    }
    if constexpr (!TILE)
        rmsnorm_block_kernel<DT, ADD, O16><<<dim3((unsigned)rows), dim3(256), 0, st>>>(out, x, y, w, rows, dim, ld_x,
                                                                                       ld_y, ld_out, eps);
    return launch_status("rmsnorm");
}

template <bool ADD, bool O16 = false, bool TILE = false>
static int launch_rmsnorm(void* out, float* x, const float* y, const void* w, int dt, long rows,
                          int dim, long ld_x, long ld_y, long ld_out, float eps, hipStream_t st) {
    switch (dt) {
        case ANELM_F32: return launch_rmsnorm_dt<ANELM_F32, ADD, O16, TILE>(out, x, y, w, rows, dim, ld_x, ld_y, ld_out, eps, st);
        case ANELM_F16: return launch_rmsnorm_dt<ANELM_F16, ADD, O16, TILE>(out, x, y, w, rows, dim, ld_x, ld_y, ld_out, eps, st);
        case ANELM_BF16: return launch_rmsnorm_dt<ANELM_BF16, ADD, O16, TILE>(out, x, y, w, rows, dim, ld_x, ld_y, ld_out, eps, st);
        default: return fail(ANELM_ERR_INVALID, "rmsnorm: unknown weight dtype %d", dt);
    }
}

// ------------------------------------------------------- q/k norm + RoPE
// models/llm/qwen3.cpp:444-472.  Per (token, head): rmsnorm over head_dim
// with the shared gamma (ane_lm::rmsnorm(qh, qh, q_norm, hd, eps)), then the
// Qwen3 half-split rotation (qwen3.cpp:17-26):
//   v[j]'      = v[j]*c[j] - v[j+half]*s[j]
//   v[j+half]' = v[j+half]*c[j] + v[j]*s[j]
// with c/s from table row pos (0 <= pos < tab_len, qwen3.cpp:463-469) or the
// fallback angle pos*inv_freq[j] (qwen3.cpp:39-49).
//
// head_dim 128 kernel: a flat grid over every head of every token (the T*nq
// q heads, then the T*nk k heads).  A 16-lane group owns one head: lane l
// holds elements 4l..4l+3 and 64+4l..64+4l+3, so each rotation pair sits in
// one lane and the sum of squares is a 16-lane shuffle reduction.  A head is
// read once and written once (non-temporal); its token's cos/sin row and
// the gammas are shared by all heads and come from cache.
//
// HPG heads per group: group g of G handles heads g, g+G, ..., so each round
// of the grid covers consecutive heads; all loads of the HPG heads (heads,
// then positions, then the table rows that depend on them) are issued before
// the first is used, which matters when a launch is only a few rounds deep.
template <int DT, int HPG>
__global__ __launch_bounds__(256) void qknorm_rope128_kernel(
    float* q, float* k, long q_ld, long k_ld, const void* wq, const void* wk, const int32_t* pos,
    const float* cos_tab, const float* sin_tab, int tab_len, const InvFreq inv, long T, int nq,
    int nk, float eps) {
    const uint32_t nqh = (uint32_t)T * (uint32_t)nq;            // heads < 2^31 (checked on the host)
    const uint32_t heads = nqh + (uint32_t)T * (uint32_t)nk;
    const uint32_t G = gridDim.x * 16u;
    const uint32_t g = blockIdx.x * 16u + (threadIdx.x >> 4);
    const int j0 = 4 * (threadIdx.x & 15);
    float* v[HPG];
    float4 lo[HPG], hi[HPG], c[HPG], s[HPG];
    int p[HPG];
    bool isq[HPG];
#pragma unroll
    for (int i = 0; i < HPG; i++) {
        const uint32_t gh = g + (uint32_t)i * G;
        v[i] = nullptr;
        isq[i] = gh < nqh;
        lo[i] = hi[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        p[i] = 0;
        if (gh < heads) {
            uint32_t t;
            if (isq[i]) {
                t = gh / (uint32_t)nq;
                v[i] = q + (long)t * q_ld + (long)(gh - t * (uint32_t)nq) * 128;
            } else {
                const uint32_t g2 = gh - nqh;
                t = g2 / (uint32_t)nk;
                v[i] = k + (long)t * k_ld + (long)(g2 - t * (uint32_t)nk) * 128;
            }
            lo[i] = ld_nt(reinterpret_cast<const float4*>(v[i] + j0));
            hi[i] = ld_nt(reinterpret_cast<const float4*>(v[i] + 64 + j0));
            p[i] = pos[t];
        }
    }
#pragma unroll
    for (int i = 0; i < HPG; i++) rope_cs4(p[i], j0, cos_tab, sin_tab, tab_len, inv.v, c[i], s[i]);
#pragma unroll
    for (int i = 0; i < HPG; i++) {
        float4 ol, oh;   // every lane takes part (dead heads contribute zeros)
        norm_rope128<DT>(lo[i], hi[i], isq[i] ? wq : wk, c[i], s[i], j0, eps, ol, oh);
        if (v[i]) {
            st_nt(reinterpret_cast<float4*>(v[i] + j0), ol);
            st_nt(reinterpret_cast<float4*>(v[i] + 64 + j0), oh);
        }
    }
}

// The same for the common case (both gammas present, a RoPE table, nq and nk
// multiples of 8): each wave owns 8 consecutive heads, which then belong to
// one token, two per 16-lane group (heads w0+sub and w0+4+sub, so each round
// of loads covers 2 KB of contiguous heads).  The wave's token is uniform,
// so its position is a scalar load, and every load of the wave -- the gammas
// (raw bits), both heads and the table row at the clamped position -- goes
// out before the first wait.  In qknorm_rope128_kernel the position is a
// vector load behind the head loads and the gammas load inside branches;
// each of those waits is a memory round trip, and the clamped, unconditional
// form measured 52 us against 58 us at the Qwen3-8B prefill shape (81.7%
// against 73.2% of 8 TB/s).  Positions past the table overwrite the table
// values with the fallback angle in a wave-uniform branch; the arithmetic is
// norm_rope128_w's, so the bits equal qknorm_rope128_kernel's.
template <int DT>
__global__ __launch_bounds__(256) void qknorm_rope128_w8_kernel(
    float* __restrict__ q, float* __restrict__ k, long q_ld, long k_ld, const void* __restrict__ wq,
    const void* __restrict__ wk, const int32_t* __restrict__ pos, const float* __restrict__ cos_tab,
    const float* __restrict__ sin_tab, int tab_len, const InvFreq inv, long T, int nq, int nk, float eps) {
    const uint32_t nqh = (uint32_t)T * (uint32_t)nq;   // heads < 2^31 (checked on the host)
    const uint32_t heads = nqh + (uint32_t)T * (uint32_t)nk;
    const uint32_t w0 = (blockIdx.x * 4u + (threadIdx.x >> 6)) * 8u;   // the wave's first head
    if (w0 >= heads) return;   // whole wave (heads is a multiple of 8)
    const bool isq = w0 < nqh;
    uint32_t t = isq ? w0 / (uint32_t)nq : (w0 - nqh) / (uint32_t)nk;
    t = __builtin_amdgcn_readfirstlane(t);
    const int p = pos[t];
    const int j0 = 4 * (threadIdx.x & 15);
    const int sub = (threadIdx.x >> 4) & 3;
    Gamma4<DT> glo, ghi;
    glo.load(isq ? wq : wk, j0);
    ghi.load(isq ? wq : wk, j0 + 64);
    float* v[2];
    float4 lo[2], hi[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t h = w0 + (uint32_t)(4 * i + sub);
        v[i] = isq ? q + (long)t * q_ld + (long)(h - t * (uint32_t)nq) * 128
                   : k + (long)t * k_ld + (long)(h - nqh - t * (uint32_t)nk) * 128;
        lo[i] = ld_nt(reinterpret_cast<const float4*>(v[i] + j0));
        hi[i] = ld_nt(reinterpret_cast<const float4*>(v[i] + 64 + j0));
    }
    const int pr = p < 0 ? 0 : (p >= tab_len ? tab_len - 1 : p);
    float4 c = *reinterpret_cast<const float4*>(cos_tab + (long)pr * 64 + j0);
    float4 s = *reinterpret_cast<const float4*>(sin_tab + (long)pr * 64 + j0);
    if (p != pr) rope_cs4(p, j0, cos_tab, sin_tab, tab_len, inv.v, c, s);   // past the table: the fallback angle
    const float4 wl = glo.get(), wh = ghi.get();
#pragma unroll
    for (int i = 0; i < 2; i++) {
        float4 ol, oh;
        norm_rope128_w(lo[i], hi[i], true, wl, wh, c, s, eps, ol, oh);
        st_nt(reinterpret_cast<float4*>(v[i] + j0), ol);
        st_nt(reinterpret_cast<float4*>(v[i] + 64 + j0), oh);
    }
}

// The decode step's q/k norm + RoPE and KV ring append in one launch
// (qwen3.cpp:444-488): token b of sequence b, one workgroup per sequence.
// Groups of 16 lanes take the heads in turn (q heads, then k heads); q and k
// are rewritten in place as anelm_qknorm_rope does, and k, with v copied as
// it is, also goes to the ring slot that anelm_kv_ring_append would pick.
// The ring state is read and advanced by one lane while the first heads'
// loads are in flight.
template <int DT>
__global__ __launch_bounds__(1024) void qknorm_rope_append128_kernel(
    float* q, float* k, const float* v, long q_ld, long k_ld, long v_ld, const void* wq, const void* wk,
    const int32_t* pos, const float* cos_tab, const float* sin_tab, int tab_len, const InvFreq inv, int nq, int nk,
    float eps, float* kc, float* vc, int32_t* rs, int32_t* rl, int cap, long seq_stride) {
    __shared__ int s_slot;
    const long b = blockIdx.x;
    const int grp = threadIdx.x >> 4, ngrp = blockDim.x >> 4;
    const int j0 = 4 * (threadIdx.x & 15);
    const int nh = nq + nk;
    auto head = [&](int hh) {
        return hh < nq ? q + b * q_ld + (long)hh * 128 : k + b * k_ld + (long)(hh - nq) * 128;
    };
    float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi = lo;
    if (grp < nh) {
        lo = ld_nt(reinterpret_cast<const float4*>(head(grp) + j0));
        hi = ld_nt(reinterpret_cast<const float4*>(head(grp) + 64 + j0));
    }
    if (threadIdx.x == 0) s_slot = ring_advance(rs + b, rl + b, cap);
    float4 c, s;
    rope_cs4(pos[b], j0, cos_tab, sin_tab, tab_len, inv.v, c, s);
    __syncthreads();
    const long row = (long)nk * 128;
    float* kd = kc + b * seq_stride + (long)s_slot * row;
    float4* vd = reinterpret_cast<float4*>(vc + b * seq_stride + (long)s_slot * row);
    const float4* vs = reinterpret_cast<const float4*>(v + b * v_ld);
    for (int i = threadIdx.x; i < nk * 32; i += blockDim.x) vd[i] = vs[i];
    for (int hh = grp; hh < nh; hh += ngrp) {   // uniform within the 16-lane group
        if (hh != grp) {
            lo = ld_nt(reinterpret_cast<const float4*>(head(hh) + j0));
            hi = ld_nt(reinterpret_cast<const float4*>(head(hh) + 64 + j0));
        }
        float4 ol, oh;
        norm_rope128<DT>(lo, hi, hh < nq ? wq : wk, c, s, j0, eps, ol, oh);
        float* dst = head(hh);
        *reinterpret_cast<float4*>(dst + j0) = ol;
        *reinterpret_cast<float4*>(dst + 64 + j0) = oh;
        if (hh >= nq) {
            float* kr = kd + (long)(hh - nq) * 128;
            *reinterpret_cast<float4*>(kr + j0) = ol;
            *reinterpret_cast<float4*>(kr + 64 + j0) = oh;
        }
    }
}

// Any even head_dim <= 1024: one wave per (token, head), two passes.
template <int DT>
__global__ __launch_bounds__(256) void qknorm_rope_generic_kernel(
    float* q, float* k, long q_ld, long k_ld, const void* wq, const void* wk, const int32_t* pos,
    const float* cos_tab, const float* sin_tab, int tab_len, const InvFreq inv, long T, int nq,
    int nk, int head_dim, float eps) {
    const int lane = threadIdx.x & 63;
    const int nh = nq + nk;
    const long gid = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gid >= T * nh) return;
    const long t = gid / nh;
    const int h = (int)(gid % nh);
    const bool isq = h < nq;
    float* v = isq ? q + t * q_ld + (long)h * head_dim : k + t * k_ld + (long)(h - nq) * head_dim;
    const void* w = isq ? wq : wk;
    const int half = head_dim / 2;
    float sc = 1.0f;
    if (w) {
        float ss = 0.f;
        for (int j = lane; j < head_dim; j += 64) ss = fmaf(v[j], v[j], ss);
        ss = wave_sum(ss);
        sc = 1.0f / sqrtf(ss / (float)head_dim + eps);
    }
    const int p = pos[t];
    const bool tab = p >= 0 && p < tab_len;
    for (int j = lane; j < half; j += 64) {
        float a = v[j], b = v[j + half];
        if (w) {
            a = (a * sc) * load_w<DT>(w, j);
            b = (b * sc) * load_w<DT>(w, j + half);
        }
        float cc, ssn;
        if (tab) {
            cc = cos_tab[(long)p * half + j];
            ssn = sin_tab[(long)p * half + j];
        } else {
            const float ang = (float)p * inv.v[j];
            cc = cosf(ang);
            ssn = sinf(ang);
        }
        v[j] = a * cc - b * ssn;
        v[j + half] = b * cc + a * ssn;
    }
}

// core/cpu_ops.cpp:56-80 for one token.  Table path: half-split over
// rot_dim; fallback: adjacent pairs (2i, 2i+1), as the reference does.
__global__ __launch_bounds__(256) void rope_cached_kernel(float* q, float* k, int nq, int nk,
                                                          int q_stride, int k_stride, int rot_dim,
                                                          int pos, const float* cos_row,
                                                          const float* sin_row, const InvFreq inv) {
    const int lane = threadIdx.x & 63;
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (h >= nq + nk) return;
    float* v = h < nq ? q + (long)h * q_stride : k + (long)(h - nq) * k_stride;
    const int half = rot_dim / 2;
    for (int j = lane; j < half; j += 64) {
        if (cos_row) {
            const float c = cos_row[j], s = sin_row[j];
            const float a = v[j], b = v[j + half];
            v[j] = a * c - b * s;
            v[j + half] = b * c + a * s;
        } else {
            const float ang = (float)pos * inv.v[j];
            const float c = cosf(ang), s = sinf(ang);
            const float a = v[2 * j], b = v[2 * j + 1];
            v[2 * j] = a * c - b * s;
            v[2 * j + 1] = a * s + b * c;
        }
    }
}

// models/llm/qwen3.cpp:210-218: cos/sin of the fp32 angle (float)pos*inv[j].
__global__ __launch_bounds__(256) void rope_table_kernel(float* cos_tab, float* sin_tab, int n_pos,
                                                         int half, const InvFreq inv) {
    const long n = (long)n_pos * half;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const int p = (int)(i / half);
        const int j = (int)(i % half);
        const float ang = (float)p * inv.v[j];
        cos_tab[i] = cosf(ang);
        sin_tab[i] = sinf(ang);
    }
}

}  // namespace anelm

using namespace anelm;

extern "C" int anelm_rmsnorm(float* out, const float* x, const void* w, int w_dtype, long rows,
                             int dim, long ld_x, long ld_out, float eps, void* stream) {
    if (!out || !x || !w) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm: null pointer");
    if (rows <= 0 || dim <= 0) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm: rows=%ld dim=%d", rows, dim);
    if (ld_x < dim || ld_out < dim) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm: ld < dim");
    if (rows > 0x7FFFFFFFL) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm: too many rows");
    clear_error();
    return launch_rmsnorm<false>(out, const_cast<float*>(x), nullptr, w, w_dtype, rows, dim, ld_x, 0,
                                 ld_out, eps, as_stream(stream));
}

extern "C" int anelm_rmsnorm_geometry(long rows, int dim, int* float4_per_lane, int* threads) {
    if (!float4_per_lane || !threads) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_geometry: null pointer");
    if (rows <= 0 || dim <= 0) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_geometry: rows=%ld dim=%d", rows, dim);
    clear_error();
    if (dim % 4 == 0 && dim / 4 <= 1024 * 4) {
        rms_row_geometry(rows, dim / 4, *float4_per_lane, *threads);
    } else {
        *float4_per_lane = 0;   // the any-shape kernel: 256 threads, two passes
        *threads = 256;
    }
    return ANELM_OK;
}

extern "C" int anelm_rmsnorm_f16(uint16_t* out16, const float* x, const void* w, int w_dtype, long rows, int dim,
                                 long ld_x, long ld_out, float eps, void* stream) {
    if (!out16 || !x || !w) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16: null pointer");
    if (rows <= 0 || dim <= 0) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16: rows=%ld dim=%d", rows, dim);
    if (ld_x < dim || ld_out < dim) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16: ld < dim");
    if (rows > 0x7FFFFFFFL) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16: too many rows");
    const uintptr_t o0 = reinterpret_cast<uintptr_t>(out16), x0 = reinterpret_cast<uintptr_t>(x);
    if (o0 < x0 + (uintptr_t)((rows - 1) * ld_x + dim) * 4u && x0 < o0 + (uintptr_t)((rows - 1) * ld_out + dim) * 2u)
        return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16: out16 overlaps x");
    clear_error();
    return launch_rmsnorm<false, true>(out16, const_cast<float*>(x), nullptr, w, w_dtype, rows, dim, ld_x, 0, ld_out,
                                       eps, as_stream(stream));
}

extern "C" int anelm_rmsnorm_f16_tiled(uint16_t* out_t, const float* x, const void* w, int w_dtype, long rows, int dim,
                                       long ld_x, float eps, void* stream) {
    if (!out_t || !x || !w) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16_tiled: null pointer");
    if (rows <= 0 || dim <= 0 || dim % 32 != 0)
        return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16_tiled: rows=%ld dim=%d (a multiple of 32)", rows, dim);
    if (ld_x < dim) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16_tiled: ld_x < dim");
    if (rows > 0x7FFFFFFFL) return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16_tiled: too many rows");
    const size_t out_bytes = (size_t)((rows + 15) / 16) * 16 * (size_t)dim * 2u;
    const uintptr_t o0 = reinterpret_cast<uintptr_t>(out_t), x0 = reinterpret_cast<uintptr_t>(x);
    if (o0 < x0 + (uintptr_t)((rows - 1) * ld_x + dim) * 4u && x0 < o0 + out_bytes)
        return fail(ANELM_ERR_INVALID, "anelm_rmsnorm_f16_tiled: out_t overlaps x");
    clear_error();
    return launch_rmsnorm<false, true, true>(out_t, const_cast<float*>(x), nullptr, w, w_dtype, rows, dim, ld_x, 0, dim,
                                             eps, as_stream(stream));
}

extern "C" int anelm_add_rmsnorm(float* x, const float* y, float* out, const void* w, int w_dtype,
                                 long rows, int dim, long ld_x, long ld_y, long ld_out, float eps,
                                 void* stream) {
    if (!out || !x || !y || !w) return fail(ANELM_ERR_INVALID, "anelm_add_rmsnorm: null pointer");
    if (rows <= 0 || dim <= 0) return fail(ANELM_ERR_INVALID, "anelm_add_rmsnorm: rows=%ld dim=%d", rows, dim);
    if (ld_x < dim || ld_y < dim || ld_out < dim) return fail(ANELM_ERR_INVALID, "anelm_add_rmsnorm: ld < dim");
    if (out == x) return fail(ANELM_ERR_INVALID, "anelm_add_rmsnorm: out must not alias x");
    if (rows > 0x7FFFFFFFL) return fail(ANELM_ERR_INVALID, "anelm_add_rmsnorm: too many rows");
    clear_error();
    return launch_rmsnorm<true>(out, x, y, w, w_dtype, rows, dim, ld_x, ld_y, ld_out, eps,
                                as_stream(stream));
}

template <int DT>
static int launch_qknorm(float* q, float* k, long q_ld, long k_ld, const void* wq, const void* wk,
                         const int32_t* pos, const float* cos_tab, const float* sin_tab, int tab_len,
                         const InvFreq& inv, long T, int nq, int nk, int head_dim, float eps,
                         hipStream_t st) {
    const bool fast = head_dim == 128 && aligned16(q) && aligned16(k) && q_ld % 4 == 0 &&
                      k_ld % 4 == 0 && (tab_len == 0 || (aligned16(cos_tab) && aligned16(sin_tab))) &&
                      (!wq || (DT == ANELM_F32 ? aligned16(wq) : aligned8(wq))) &&
                      (!wk || (DT == ANELM_F32 ? aligned16(wk) : aligned8(wk)));
    if (fast && wq && wk && tab_len > 0 && nq % 8 == 0 && nk % 8 == 0) {
        const long waves = T * (nq + nk) / 8;
        qknorm_rope128_w8_kernel<DT><<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st>>>(
            q, k, q_ld, k_ld, wq, wk, pos, cos_tab, sin_tab, tab_len, inv, T, nq, nk, eps);
    } else if (fast) {
        // one head per group measured fastest at every shape from T=1 to the
        // 8B prefill (two or four per group: equal at best, slower at decode)
        const long heads = T * (nq + nk);
        const unsigned blocks = (unsigned)((heads * 16 + 255) / 256);
        qknorm_rope128_kernel<DT, 1><<<dim3(blocks), dim3(256), 0, st>>>(
            q, k, q_ld, k_ld, wq, wk, pos, cos_tab, sin_tab, tab_len, inv, T, nq, nk, eps);
    } else {
        const long waves = T * (nq + nk);
        qknorm_rope_generic_kernel<DT><<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st>>>(
            q, k, q_ld, k_ld, wq, wk, pos, cos_tab, sin_tab, tab_len, inv, T, nq, nk, head_dim, eps);
    }
    return launch_status("qknorm_rope");
}

extern "C" int anelm_qknorm_rope(float* q, float* k, long q_ld, long k_ld, const void* wq,
                                 const void* wk, int w_dtype, const int32_t* pos,
                                 const float* cos_tab, const float* sin_tab, int tab_len, float theta,
                                 long T, int nq, int nk, int head_dim, float eps, void* stream) {
    if (!pos) return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: null pos");
    if (T <= 0 || nq < 0 || nk < 0 || nq + nk == 0) return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: empty");
    if ((nq > 0 && !q) || (nk > 0 && !k)) return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: null q/k");
    if (head_dim <= 0 || head_dim % 2 || head_dim > 1024) return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: head_dim %d", head_dim);
    if ((nq > 0 && q_ld < (long)nq * head_dim) || (nk > 0 && k_ld < (long)nk * head_dim))
        return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: token stride too small");
    if (tab_len < 0 || (tab_len > 0 && (!cos_tab || !sin_tab))) return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: table");
    if (T > (1L << 40) || T * (nq + nk) > 0x7FFFFFFFL) return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: too large");
    if (w_dtype < ANELM_F32 || w_dtype > ANELM_BF16) return fail(ANELM_ERR_INVALID, "anelm_qknorm_rope: dtype");
    InvFreq inv;
    rope_inv_freq(&inv, head_dim, theta);
    clear_error();
    hipStream_t st = as_stream(stream);
    if (nq == 0) q = k;  // never dereferenced, keeps pointer arithmetic defined
    if (nk == 0) k = q;
    switch (w_dtype) {
        case ANELM_F32: return launch_qknorm<ANELM_F32>(q, k, q_ld, k_ld, wq, wk, pos, cos_tab, sin_tab, tab_len, inv, T, nq, nk, head_dim, eps, st);
        case ANELM_F16: return launch_qknorm<ANELM_F16>(q, k, q_ld, k_ld, wq, wk, pos, cos_tab, sin_tab, tab_len, inv, T, nq, nk, head_dim, eps, st);
        default: return launch_qknorm<ANELM_BF16>(q, k, q_ld, k_ld, wq, wk, pos, cos_tab, sin_tab, tab_len, inv, T, nq, nk, head_dim, eps, st);
    }
}

extern "C" int anelm_qknorm_rope_append(float* q, float* k, const float* v, long q_ld, long k_ld, long v_ld,
                                        const void* wq, const void* wk, int w_dtype, const int32_t* pos,
                                        const float* cos_tab, const float* sin_tab, int tab_len, float theta,
                                        long batch, int nq, int nk, float eps, float* k_cache, float* v_cache,
                                        int32_t* ring_start, int32_t* ring_len, int capacity, long cache_seq_stride,
                                        void* stream) {
    const char* fn = "anelm_qknorm_rope_append";
    if (!k || !v || !pos || !k_cache || !v_cache || !ring_start || !ring_len || (nq > 0 && !q))
        return fail(ANELM_ERR_INVALID, "%s: null pointer", fn);
    if (batch <= 0 || batch > 0x7FFFFFFFL || nq < 0 || nk <= 0 || capacity <= 0 || nq + nk > (1 << 20))
        return fail(ANELM_ERR_INVALID, "%s: bad sizes", fn);
    const long row = (long)nk * 128;
    if (batch > 1 && ((nq > 0 && q_ld < (long)nq * 128) || k_ld < row || v_ld < row ||
                      cache_seq_stride < (long)capacity * row))
        return fail(ANELM_ERR_INVALID, "%s: strides overlap", fn);
    if (tab_len < 0 || (tab_len > 0 && (!cos_tab || !sin_tab))) return fail(ANELM_ERR_INVALID, "%s: table", fn);
    if (w_dtype < ANELM_F32 || w_dtype > ANELM_BF16) return fail(ANELM_ERR_INVALID, "%s: dtype", fn);
    const bool wal = w_dtype == ANELM_F32 ? (!wq || aligned16(wq)) && (!wk || aligned16(wk))
                                          : (!wq || aligned8(wq)) && (!wk || aligned8(wk));
    if (!aligned16(k) || !aligned16(v) || (nq > 0 && !aligned16(q)) || !aligned16(k_cache) || !aligned16(v_cache) ||
        (q_ld | k_ld | v_ld | cache_seq_stride) & 3 || !wal ||
        (tab_len > 0 && (!aligned16(cos_tab) || !aligned16(sin_tab))))
        return fail(ANELM_ERR_INVALID, "%s: needs 16-byte aligned rows (strides multiples of 4)", fn);
    InvFreq inv;
    rope_inv_freq(&inv, 128, theta);
    clear_error();
    if (nq == 0) q = k;  // never dereferenced
    const int threads = (int)std::min<long>(1024, ((long)(nq + nk) * 16 + 63) / 64 * 64);
    const dim3 grid((unsigned)batch), block((unsigned)threads);
    hipStream_t st = as_stream(stream);
#define LAUNCH(DT)                                                                                            \
    qknorm_rope_append128_kernel<DT><<<grid, block, 0, st>>>(q, k, v, q_ld, k_ld, v_ld, wq, wk, pos, cos_tab, \
                                                             sin_tab, tab_len, inv, nq, nk, eps, k_cache,     \
                                                             v_cache, ring_start, ring_len, capacity,         \
                                                             cache_seq_stride)
    switch (w_dtype) {
        case ANELM_F32: LAUNCH(ANELM_F32); break;
        case ANELM_F16: LAUNCH(ANELM_F16); break;
        default: LAUNCH(ANELM_BF16); break;
    }
#undef LAUNCH
    return launch_status("qknorm_rope_append");
}

extern "C" int anelm_rope_cached(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                                 int q_head_stride, int k_head_stride, int rot_dim, int pos,
                                 float theta, const float* cos_row, const float* sin_row,
                                 void* stream) {
    if (n_q_heads < 0 || n_kv_heads < 0 || n_q_heads + n_kv_heads == 0) return fail(ANELM_ERR_INVALID, "anelm_rope_cached: no heads");
    if ((n_q_heads > 0 && !q) || (n_kv_heads > 0 && !k)) return fail(ANELM_ERR_INVALID, "anelm_rope_cached: null q/k");
    if (rot_dim <= 0 || rot_dim % 2 || rot_dim > 1024 || rot_dim > head_dim) return fail(ANELM_ERR_INVALID, "anelm_rope_cached: rot_dim %d", rot_dim);
    if ((cos_row == nullptr) != (sin_row == nullptr)) return fail(ANELM_ERR_INVALID, "anelm_rope_cached: one of cos/sin row missing");
    InvFreq inv;
    rope_inv_freq(&inv, rot_dim, theta);
    clear_error();
    if (n_q_heads == 0) q = k;
    if (n_kv_heads == 0) k = q;
    const int nh = n_q_heads + n_kv_heads;
    rope_cached_kernel<<<dim3((unsigned)((nh + 3) / 4)), dim3(256), 0, as_stream(stream)>>>(
        q, k, n_q_heads, n_kv_heads, q_head_stride, k_head_stride, rot_dim, pos, cos_row, sin_row, inv);
    return launch_status("rope_cached");
}

extern "C" int anelm_rope_table(float* cos_tab, float* sin_tab, int n_pos, int rot_dim, float theta,
                                void* stream) {
    if (!cos_tab || !sin_tab) return fail(ANELM_ERR_INVALID, "anelm_rope_table: null pointer");
    if (n_pos <= 0 || rot_dim <= 0 || rot_dim % 2 || rot_dim > 1024) return fail(ANELM_ERR_INVALID, "anelm_rope_table: n_pos=%d rot_dim=%d", n_pos, rot_dim);
    InvFreq inv;
    rope_inv_freq(&inv, rot_dim, theta);
    clear_error();
    const long n = (long)n_pos * (rot_dim / 2);
    long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    rope_table_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(cos_tab, sin_tab, n_pos, rot_dim / 2, inv);
    return launch_status("rope_table");
}
