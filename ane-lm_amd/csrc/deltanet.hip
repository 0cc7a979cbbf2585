// Qwen3.5 linear-attention (DeltaNet) ops and matvec for gfx950: gated
// RMSNorm, L2 normalisation, the causal conv1d state update, the delta-rule
// state step, and y = W x.  Replaces core/cpu_ops.cpp:33-39 and :100-171 as
// models/llm/qwen3_5.cpp:493-549 calls them, batched over sequences.
//
// All are HBM- or latency-bound.  The dominant one at batch is the state
// step: each (sequence, value head) state [key_dim, value_dim] is read once
// and written once per token, held in registers in between.
#include <cmath>

#include "anelm_common.hpp"

namespace anelm {
namespace {

constexpr int kRowThreads = 256;  // 4 rows per workgroup, one wave each

// ------------------------------------------------------------ gated RMSNorm
// core/cpu_ops.cpp:33-39: out = rmsnorm(x)*w (cpu_ops.cpp:25-31 rounding
// steps), then out = out / (1 + expf(-z)), then out *= z.
// Vector v = (row, head) of rows x heads, at row*ld + head*dim.
template <int DT>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_gated_kernel(float* out, const float* x, const float* z,
                                                                    const void* w, long rows, int heads, int dim,
                                                                    long ld_x, long ld_z, long ld_out, float eps) {
    const long vi = (long)blockIdx.x * (kRowThreads / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (vi >= rows * heads) return;
    const long row = vi / heads, h = vi % heads;
    const float* xr = x + row * ld_x + h * dim;
    const float* zr = z + row * ld_z + h * dim;
    float* orow = out + row * ld_out + h * dim;
    float ss = 0.0f;
    for (int i = lane; i < dim; i += kWave) ss = fmaf(xr[i], xr[i], ss);
    ss = wave_sum(ss);
    const float s = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = lane; i < dim; i += kWave) {
        float o = (xr[i] * s) * load_w<DT>(w, i);
        const float zi = zr[i];
        o = o / (1.0f + expf(-zi));
        orow[i] = o * zi;
    }
}

// ------------------------------------------------------------ L2 normalise
// core/cpu_ops.cpp:105-110: x *= 1/sqrtf(sum x^2 + 1e-12); then x *= scale
// (the caller's separate vDSP_vsmul, qwen3_5.cpp:530-531; 1 is exact).
__global__ __launch_bounds__(kRowThreads) void l2_normalize_kernel(float* x, long rows, int heads, int dim, long ld,
                                                                   float scale) {
    const long vi = (long)blockIdx.x * (kRowThreads / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (vi >= rows * heads) return;
    float* xr = x + (vi / heads) * ld + (vi % heads) * dim;
    float ss = 0.0f;
    for (int i = lane; i < dim; i += kWave) ss = fmaf(xr[i], xr[i], ss);
    ss = wave_sum(ss);
    const float norm = 1.0f / sqrtf(ss + 1e-12f);
    for (int i = lane; i < dim; i += kWave) xr[i] = (xr[i] * norm) * scale;
}

// ------------------------------------------------------------ conv1d update
// core/cpu_ops.cpp:112-150, one workgroup per sequence: every thread reads
// the sequence's ring position before the barrier, thread 0 advances it
// after.  Fused multiply-adds in the reference's order, so results are
// bit-identical to the oracle's.
__global__ __launch_bounds__(1024) void conv1d_update_kernel(float* y, float* state, int32_t* state_pos,
                                                             const float* x, const float* w, int channels,
                                                             int kernel_size, long ld_x, long ld_y,
                                                             long state_stride) {
    const long b = blockIdx.x;
    const int state_len = kernel_size - 1;
    float* st = state + b * state_stride;
    const float* xb = x + b * ld_x;
    float* yb = y + b * ld_y;
    int pos;
    if (kernel_size == 4) {
        // the common case: every load of a batch of channels is issued
        // before the first is used, at a clamped channel (unconditional);
        // the three ring slots are loaded at fixed offsets and picked by the
        // ring position afterwards (oldest first: pos, pos+1, pos+2 mod 3),
        // and the position is loaded after the first batch's loads (a vector
        // load: as a scalar load it was waited for before any other went out)
        constexpr int kB = 8;
        float t0[kB], t1[kB], t2[kB], xc[kB];
        float4 wc[kB];
        auto load = [&](int c0) {
#pragma unroll
            for (int u = 0; u < kB; u++) {
                const int c = c0 + u * 1024 < channels ? c0 + u * 1024 : channels - 1;
                const float* sc = st + (long)c * 3;
                t0[u] = sc[0];
                t1[u] = sc[1];
                t2[u] = sc[2];
                xc[u] = xb[c];
                wc[u] = *reinterpret_cast<const float4*>(w + (long)c * 4);
            }
        };
        auto compute = [&](int c0, int p) {
#pragma unroll
            for (int u = 0; u < kB; u++) {
                const int c = c0 + u * 1024;
                if (c < channels) {
                    const float o0 = p == 0 ? t0[u] : (p == 1 ? t1[u] : t2[u]);
                    const float o1 = p == 0 ? t1[u] : (p == 1 ? t2[u] : t0[u]);
                    const float o2 = p == 0 ? t2[u] : (p == 1 ? t0[u] : t1[u]);
                    const float sum = fmaf(o2, wc[u].z, fmaf(o1, wc[u].y, fmaf(o0, wc[u].x, 0.0f)));
                    yb[c] = fmaf(xc[u], wc[u].w, sum);
                    st[(long)c * 3 + p] = xc[u];
                }
            }
        };
        load((int)threadIdx.x);
        pos = __hip_atomic_load(state_pos + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_sched_barrier(0);
        pos = pos < 0 ? 0 : (pos >= 3 ? 0 : pos);   // keeps every access in the ring
        compute((int)threadIdx.x, pos);
        for (int c0 = (int)threadIdx.x + kB * 1024; c0 < channels; c0 += kB * 1024) {
            load(c0);
            compute(c0, pos);
        }
    } else {
        pos = state_pos[b];
        pos = pos < 0 ? 0 : (pos >= state_len ? 0 : pos);   // keeps every access in the ring
        for (int c = threadIdx.x; c < channels; c += blockDim.x) {
            float* sc = st + (long)c * state_len;
            const float* wc = w + (long)c * kernel_size;
            float sum = 0.0f;
            for (int j = 0; j < state_len; j++) {
                int idx = pos + j;
                if (idx >= state_len) idx -= state_len;
                sum = fmaf(sc[idx], wc[j], sum);
            }
            const float xv = xb[c];
            yb[c] = fmaf(xv, wc[state_len], sum);
            sc[pos] = xv;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) state_pos[b] = pos + 1 == state_len ? 0 : pos + 1;
}

// ---------------------------------------- conv1d + SiLU + q/k L2 normalise
// The decode step's qwen3_5.cpp:513-531 for kernel size 4 and 128-wide key
// heads, one workgroup per sequence: channels are [q heads | k heads | v],
// each q/k head 128 channels.  Wave w takes the 128-channel blocks w, w+nw,
// ... (nw waves, at most 16); lane l computes channels 128*blk + l and 128*blk + 64 + l, so every
// value is produced by the same operations in the same order as
// anelm_conv1d_update, anelm_silu and anelm_l2_normalize (whose wave per
// head sums element l, then l + 64, in lane l) produce it one after the other.
// One channel's kernel-4 convolution: the three ring taps oldest first
// (s0 at the ring position, then s1, s2), then the new input xc.
__device__ __forceinline__ float conv4(float s0, float s1, float s2, float xc, float4 wc) {
    const float sum = fmaf(s2, wc.z, fmaf(s1, wc.y, fmaf(s0, wc.x, 0.0f)));
    return fmaf(xc, wc.w, sum);
}

// Each wave takes the 128-channel blocks wv, wv + nw, ... of its sequence,
// BPW at a time: the loads of all BPW blocks (clamped to the last block, so
// they stay unconditional) go out before the first block's arithmetic, and
// a channel's three ring taps are loaded at fixed offsets and picked by the
// ring position afterwards.  The ring position is loaded after the first
// pass's loads (a vector load: a scalar one was waited for, with the kernel
// arguments, before any state load went out), so a sequence up to 64 blocks
// costs one memory round trip.
template <int BPW>
struct ConvPass {
    float xs[BPW][2], t0[BPW][2], t1[BPW][2], t2[BPW][2];
    float4 wc[BPW][2];
};

template <int BPW>
__global__ __launch_bounds__(1024) void conv_silu_l2_kernel(float* y, float* state, int32_t* state_pos, const float* x,
                                                            const float* w, int channels, int nq_ch, long ld_x,
                                                            long ld_y, long state_stride, float q_scale) {
    const long b = blockIdx.x;
    float* st = state + b * state_stride;
    const float* xb = x + b * ld_x;
    float* yb = y + b * ld_y;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int nblk = channels / 128;
    auto load = [&](ConvPass<BPW>& P, int base) {
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int blk = base + j * nw + wv;
            const long bc = blk < nblk ? blk : nblk - 1;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const long c = bc * 128 + lane + 64 * h;
                P.xs[j][h] = xb[c];
                P.wc[j][h] = *reinterpret_cast<const float4*>(w + c * 4);
                P.t0[j][h] = st[c * 3];
                P.t1[j][h] = st[c * 3 + 1];
                P.t2[j][h] = st[c * 3 + 2];
            }
        }
    };
    auto compute = [&](const ConvPass<BPW>& P, int base, int pos) {
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int blk = base + j * nw + wv;
            if (blk >= nblk) break;   // uniform within the wave
            float yv[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const long c = (long)blk * 128 + lane + 64 * h;
                // taps oldest first: ring slots pos, pos + 1, pos + 2 (mod 3)
                const float a0 = P.t0[j][h], a1 = P.t1[j][h], a2 = P.t2[j][h];
                const float o0 = pos == 0 ? a0 : (pos == 1 ? a1 : a2);
                const float o1 = pos == 0 ? a1 : (pos == 1 ? a2 : a0);
                const float o2 = pos == 0 ? a2 : (pos == 1 ? a0 : a1);
                const float yc = conv4(o0, o1, o2, P.xs[j][h], P.wc[j][h]);
                st[c * 3 + pos] = P.xs[j][h];
                yv[h] = yc / (expf(-yc) + 1.0f);   // SiLU, qwen3_5.cpp:514
            }
            if (blk * 128 < 2 * nq_ch) {   // a q or k head: L2 normalise (x scale)
                float ss = fmaf(yv[0], yv[0], 0.0f);
                ss = fmaf(yv[1], yv[1], ss);
                ss = wave_sum(ss);
                const float norm = 1.0f / sqrtf(ss + 1e-12f);
                const float scale = blk * 128 < nq_ch ? q_scale : 1.0f;
                yv[0] = (yv[0] * norm) * scale;
                yv[1] = (yv[1] * norm) * scale;
            }
            yb[(long)blk * 128 + lane] = yv[0];
            yb[(long)blk * 128 + lane + 64] = yv[1];
        }
    };
    ConvPass<BPW> P;
    load(P, 0);
    int pos = __hip_atomic_load(state_pos + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_sched_barrier(0);
    pos = pos < 0 ? 0 : (pos >= 3 ? 0 : pos);   // keeps every access in the ring
    compute(P, 0, pos);
    for (int base = nw * BPW; base < nblk; base += nw * BPW) {   // past 64 blocks: more passes
        load(P, base);
        compute(P, base, pos);
    }
    __syncthreads();
    if (threadIdx.x == 0) state_pos[b] = pos + 1 == 3 ? 0 : pos + 1;
}

// ------------------------------------------------------------ delta-rule step
// core/cpu_ops.cpp:152-171 for one (sequence, value head) per workgroup:
//   Sk = S^T k;  delta = v - Sk;  S = decay*S + beta*k*delta^T;  y = S^T q.
// 256 threads: VD/4 column groups of 4 columns (float4) x RG row groups of
// RPT consecutive rows.  The state is read once (non-temporal), kept in
// registers for both reductions and the update, and written once.
struct SsmArgs {
    float* y;
    float* state;
    const float* q;
    const float* k;
    const float* v;
    const float* decay;   // [batch * nvh]
    const float* beta;    // [batch * nvh]
    int nvh, nkh;         // value heads, key heads (value head h uses key head h / (nvh/nkh))
    long ld_qk, ld_v, ld_y, state_stride;  // per-sequence strides
    // gated RMSNorm epilogue (GATED): out = rmsnorm(y)*w / (1 + expf(-z)) * z
    const float* z;
    const void* nw;
    float* out;
    long ld_z, ld_out;
    float eps;
};

// With GATED the head's y is not stored: the epilogue applies
// anelm_rmsnorm_gated to it (qwen3_5.cpp:545-549) with that kernel's
// operations in its order (wave 0, lane l: elements l, l+64, ...) and stores
// the result.
template <int KD, int VD, int GATED = -1>
__global__ __launch_bounds__(256) void ssm_step_kernel(SsmArgs a) {
    constexpr int CG = VD / 4;          // column groups
    constexpr int RG = 256 / CG;        // row groups
    constexpr int RPT = KD / RG;        // rows per thread
    __shared__ float sk[KD], sq[KD], sdelta[VD];
    __shared__ float red[RG][VD];
    const int tid = threadIdx.x;
    const int cg = tid % CG, rg = tid / CG;
    const long bh = blockIdx.x;
    const long b = bh / a.nvh;
    const int vh = (int)(bh % a.nvh);
    const int kh = vh / (a.nvh / a.nkh);
    const float* kp = a.k + b * a.ld_qk + (long)kh * KD;
    const float* qp = a.q + b * a.ld_qk + (long)kh * KD;
    const float* vp = a.v + b * a.ld_v + (long)vh * VD;
    float* S = a.state + b * a.state_stride + (long)vh * KD * VD;
    const float decay = a.decay[bh], beta = a.beta[bh];

    float4 s[RPT];
#pragma unroll
    for (int r = 0; r < RPT; r++) s[r] = ld_nt(reinterpret_cast<const float4*>(S + (long)(rg * RPT + r) * VD) + cg);
    for (int i = tid; i < KD; i += 256) {
        sk[i] = kp[i];
        sq[i] = qp[i];
    }
    __syncthreads();
    // Sk = S^T k
    float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        const float kr = sk[rg * RPT + r];
        p.x = fmaf(s[r].x, kr, p.x);
        p.y = fmaf(s[r].y, kr, p.y);
        p.z = fmaf(s[r].z, kr, p.z);
        p.w = fmaf(s[r].w, kr, p.w);
    }
    *reinterpret_cast<float4*>(&red[rg][4 * cg]) = p;
    __syncthreads();
    for (int j = tid; j < VD; j += 256) {
        float t = red[0][j];
#pragma unroll
        for (int g = 1; g < RG; g++) t += red[g][j];
        sdelta[j] = vp[j] - t;
    }
    __syncthreads();
    // S = decay*S + beta*k*delta^T, then y = S^T q
    const float4 d = *reinterpret_cast<const float4*>(&sdelta[4 * cg]);
    p = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        const float bk = beta * sk[rg * RPT + r];
        s[r].x = fmaf(bk, d.x, s[r].x * decay);
        s[r].y = fmaf(bk, d.y, s[r].y * decay);
        s[r].z = fmaf(bk, d.z, s[r].z * decay);
        s[r].w = fmaf(bk, d.w, s[r].w * decay);
        const float qr = sq[rg * RPT + r];
        p.x = fmaf(s[r].x, qr, p.x);
        p.y = fmaf(s[r].y, qr, p.y);
        p.z = fmaf(s[r].z, qr, p.z);
        p.w = fmaf(s[r].w, qr, p.w);
        st_nt(reinterpret_cast<float4*>(S + (long)(rg * RPT + r) * VD) + cg, s[r]);
    }
    *reinterpret_cast<float4*>(&red[rg][4 * cg]) = p;   // red was last read before the previous barrier
    __syncthreads();
    if constexpr (GATED < 0) {
        float* yp = a.y + b * a.ld_y + (long)vh * VD;
        for (int j = tid; j < VD; j += 256) {
            float t = red[0][j];
#pragma unroll
            for (int g = 1; g < RG; g++) t += red[g][j];
            yp[j] = t;
        }
    } else {
        for (int j = tid; j < VD; j += 256) {   // y into sdelta (last read before the previous barrier)
            float t = red[0][j];
#pragma unroll
            for (int g = 1; g < RG; g++) t += red[g][j];
            sdelta[j] = t;
        }
        __syncthreads();
        if (tid < kWave) {
            float ss = 0.0f;
            for (int i = tid; i < VD; i += kWave) ss = fmaf(sdelta[i], sdelta[i], ss);
            ss = wave_sum(ss);
            const float sc = 1.0f / sqrtf(ss / (float)VD + a.eps);
            const float* zr = a.z + b * a.ld_z + (long)vh * VD;
            float* orow = a.out + b * a.ld_out + (long)vh * VD;
            for (int i = tid; i < VD; i += kWave) {
                float o = (sdelta[i] * sc) * load_w<GATED>(a.nw, i);
                const float zi = zr[i];
                o = o / (1.0f + expf(-zi));
                orow[i] = o * zi;
            }
        }
    }
}

// ------------------------------------- conv + SiLU + L2 norm + delta-rule step
// qwen3_5.cpp:513-549 for one (sequence, head) per workgroup, with 128-wide
// key and value heads and one key head per value head: waves 0, 1 and 2
// compute the conv1d, SiLU (and for q and k the L2 norm, q scaled) of the
// head's own q, k and v channels -- the operations and lane mapping of
// conv_silu_l2_kernel, lane l on channels l and l + 64 -- and update those
// channels' ring slots; then the delta-rule step and the gated RMSNorm of
// ssm_step_kernel<128, 128, GATED> run on them from LDS.  The state loads go
// out first, the conv's loads with them.  No workgroup touches another's
// channels, so each (sequence, head) keeps its own ring position
// (head_pos[b * nh + h]), advanced by its workgroup.
struct ConvSsmArgs {
    float* state;
    float* conv_state;
    int32_t* head_pos;
    const float* x;
    const float* conv_w;
    const float* decay;
    const float* beta;
    const float* z;
    const void* nw;
    float* out;
    int nh;
    long ld_x, ld_z, ld_out, state_stride, conv_stride;
    float q_scale, eps;
};

template <int GATED>
__global__ __launch_bounds__(256) void conv_ssm_kernel(ConvSsmArgs a) {
    constexpr int KD = 128, VD = 128;
    constexpr int CG = VD / 4, RG = 256 / CG, RPT = KD / RG;
    __shared__ float sk[KD], sq[KD], sv[VD], sdelta[VD];
    __shared__ float red[RG][VD];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int cg = tid % CG, rg = tid / CG;
    const long bh = blockIdx.x;
    const long b = bh / a.nh;
    const int h = (int)(bh % a.nh);
    const long nq_ch = (long)a.nh * 128;
    float* S = a.state + b * a.state_stride + (long)h * KD * VD;
    float4 s[RPT];
#pragma unroll
    for (int r = 0; r < RPT; r++) s[r] = ld_nt(reinterpret_cast<const float4*>(S + (long)(rg * RPT + r) * VD) + cg);
    // this wave's 128 channels: q (wave 0), k (wave 1) or v (wave 2) of head
    // h.  Wave 3 issues the same loads unconditionally (a load in a branch is
    // waited for at the branch's end) at wave 2's channels and discards them;
    // its ring taps come from the read-only weights (in bounds: c*3 + 2 <
    // 4*channels), so it reads nothing that wave 2 writes.
    const int part = wv < 3 ? wv : 2;
    const long cb = (long)part * nq_ch + (long)h * 128;
    float* st = a.conv_state + b * a.conv_stride;
    const float* taps = wv < 3 ? st : a.conv_w;
    const float* xb = a.x + b * a.ld_x;
    float xs[2], t0[2], t1[2], t2[2];
    float4 wc[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const long c = cb + lane + 64 * u;
        xs[u] = xb[c];
        wc[u] = *reinterpret_cast<const float4*>(a.conv_w + c * 4);
        t0[u] = taps[c * 3];
        t1[u] = taps[c * 3 + 1];
        t2[u] = taps[c * 3 + 2];
    }
    int pos = __hip_atomic_load(a.head_pos + bh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float decay = a.decay[bh], beta = a.beta[bh];
    __builtin_amdgcn_sched_barrier(0);
    pos = pos < 0 ? 0 : (pos >= 3 ? 0 : pos);   // keeps every access in the ring
    if (wv < 3) {
        float yv[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const long c = cb + lane + 64 * u;
            const float o0 = pos == 0 ? t0[u] : (pos == 1 ? t1[u] : t2[u]);
            const float o1 = pos == 0 ? t1[u] : (pos == 1 ? t2[u] : t0[u]);
            const float o2 = pos == 0 ? t2[u] : (pos == 1 ? t0[u] : t1[u]);
            const float yc = conv4(o0, o1, o2, xs[u], wc[u]);
            st[c * 3 + pos] = xs[u];
            yv[u] = yc / (expf(-yc) + 1.0f);   // SiLU, qwen3_5.cpp:514
        }
        if (wv < 2) {   // q or k: L2 normalise (q scaled)
            float ss = fmaf(yv[0], yv[0], 0.0f);
            ss = fmaf(yv[1], yv[1], ss);
            ss = wave_sum(ss);
            const float norm = 1.0f / sqrtf(ss + 1e-12f);
            const float scale = wv == 0 ? a.q_scale : 1.0f;
            yv[0] = (yv[0] * norm) * scale;
            yv[1] = (yv[1] * norm) * scale;
        }
        float* dst = wv == 0 ? sq : (wv == 1 ? sk : sv);
        dst[lane] = yv[0];
        dst[lane + 64] = yv[1];
    }
    __syncthreads();   // every wave has read the ring position
    if (tid == 0) a.head_pos[bh] = pos + 1 == 3 ? 0 : pos + 1;
    // Sk = S^T k (ssm_step_kernel's operations from here on)
    float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        const float kr = sk[rg * RPT + r];
        p.x = fmaf(s[r].x, kr, p.x);
        p.y = fmaf(s[r].y, kr, p.y);
        p.z = fmaf(s[r].z, kr, p.z);
        p.w = fmaf(s[r].w, kr, p.w);
    }
    *reinterpret_cast<float4*>(&red[rg][4 * cg]) = p;
    __syncthreads();
    for (int j = tid; j < VD; j += 256) {
        float t = red[0][j];
#pragma unroll
        for (int g = 1; g < RG; g++) t += red[g][j];
        sdelta[j] = sv[j] - t;
    }
    __syncthreads();
    const float4 d = *reinterpret_cast<const float4*>(&sdelta[4 * cg]);
    p = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        const float bk = beta * sk[rg * RPT + r];
        s[r].x = fmaf(bk, d.x, s[r].x * decay);
        s[r].y = fmaf(bk, d.y, s[r].y * decay);
        s[r].z = fmaf(bk, d.z, s[r].z * decay);
        s[r].w = fmaf(bk, d.w, s[r].w * decay);
        const float qr = sq[rg * RPT + r];
        p.x = fmaf(s[r].x, qr, p.x);
        p.y = fmaf(s[r].y, qr, p.y);
        p.z = fmaf(s[r].z, qr, p.z);
        p.w = fmaf(s[r].w, qr, p.w);
        st_nt(reinterpret_cast<float4*>(S + (long)(rg * RPT + r) * VD) + cg, s[r]);
    }
    *reinterpret_cast<float4*>(&red[rg][4 * cg]) = p;   // red was last read before the previous barrier
    __syncthreads();
    for (int j = tid; j < VD; j += 256) {   // y into sdelta (last read before the previous barrier)
        float t = red[0][j];
#pragma unroll
        for (int g = 1; g < RG; g++) t += red[g][j];
        sdelta[j] = t;
    }
    __syncthreads();
    if (tid < kWave) {
        float ss = 0.0f;
        for (int i = tid; i < VD; i += kWave) ss = fmaf(sdelta[i], sdelta[i], ss);
        ss = wave_sum(ss);
        const float sc = 1.0f / sqrtf(ss / (float)VD + a.eps);
        const float* zr = a.z + b * a.ld_z + (long)h * VD;
        float* orow = a.out + b * a.ld_out + (long)h * VD;
        for (int i = tid; i < VD; i += kWave) {
            float o = (sdelta[i] * sc) * load_w<GATED>(a.nw, i);
            const float zi = zr[i];
            o = o / (1.0f + expf(-zi));
            orow[i] = o * zi;
        }
    }
}

// ------------------------------------------------------------ matvec
// core/cpu_ops.cpp:100-103: y = W x, W [out_dim, in_dim] row-major fp32.
// One wave per row; W is streamed once (non-temporal), x comes from cache.
template <bool VEC>
__global__ __launch_bounds__(kRowThreads) void matvec_kernel(float* y, const float* W, const float* x, long out_dim,
                                                             int in_dim) {
    const long row = (long)blockIdx.x * (kRowThreads / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= out_dim) return;
    const float* wr = W + row * (long)in_dim;
    float acc = 0.0f;
    if (VEC) {
        const int n4 = in_dim / 4;
        constexpr int U = 4;
        for (int c0 = 0; c0 < n4; c0 += kWave * U) {
            float4 wv[U], xv[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = c0 + u * kWave + lane;
                wv[u] = c < n4 ? ld_nt(reinterpret_cast<const float4*>(wr) + c) : make_float4(0.f, 0.f, 0.f, 0.f);
                xv[u] = c < n4 ? reinterpret_cast<const float4*>(x)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                acc = fmaf(wv[u].x, xv[u].x, acc);
                acc = fmaf(wv[u].y, xv[u].y, acc);
                acc = fmaf(wv[u].z, xv[u].z, acc);
                acc = fmaf(wv[u].w, xv[u].w, acc);
            }
        }
    } else {
        for (int c = lane; c < in_dim; c += kWave) acc = fmaf(wr[c], x[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

long row_blocks(long rows) { return (rows + kRowThreads / kWave - 1) / (kRowThreads / kWave); }

template <int KD, int VD>
void launch_ssm(const SsmArgs& a, long n, hipStream_t st, int gated_dtype = -1) {
    switch (gated_dtype) {
        case -1: hipLaunchKernelGGL((ssm_step_kernel<KD, VD>), dim3(n), dim3(256), 0, st, a); break;
        case ANELM_F32: hipLaunchKernelGGL((ssm_step_kernel<KD, VD, ANELM_F32>), dim3(n), dim3(256), 0, st, a); break;
        case ANELM_F16: hipLaunchKernelGGL((ssm_step_kernel<KD, VD, ANELM_F16>), dim3(n), dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((ssm_step_kernel<KD, VD, ANELM_BF16>), dim3(n), dim3(256), 0, st, a); break;
    }
}

int ssm_check(const char* fn, long batch, int n_heads, int n_key_heads, int key_dim, int value_dim, long ld_qk,
              long ld_v, long ld_y, long state_stride, const float* state) {
    if (batch < 0 || n_heads <= 0 || n_key_heads <= 0 || n_heads % n_key_heads)
        return fail(ANELM_ERR_INVALID, "%s: n_heads must be a positive multiple of n_key_heads", fn);
    const bool kd_ok = key_dim == 64 || key_dim == 128 || key_dim == 256;
    if (!kd_ok || (value_dim != 64 && value_dim != 128))
        return fail(ANELM_ERR_INVALID, "%s: key_dim %d / value_dim %d (64/128/256 and 64/128)", fn, key_dim, value_dim);
    if (batch > 1 && (ld_qk < (long)n_key_heads * key_dim || ld_v < (long)n_heads * value_dim ||
                      ld_y < (long)n_heads * value_dim || state_stride < (long)n_heads * key_dim * value_dim))
        return fail(ANELM_ERR_INVALID, "%s: strides overlap", fn);
    if (!aligned16(state) || (state_stride & 3)) return fail(ANELM_ERR_INVALID, "%s: state not 16-byte aligned", fn);
    return ANELM_OK;
}

int ssm_launch(const SsmArgs& a, long batch, int n_heads, int key_dim, int value_dim, int gated_dtype,
               hipStream_t st) {
    const long n = batch * n_heads;
    if (value_dim == 128) {
        if (key_dim == 64) launch_ssm<64, 128>(a, n, st, gated_dtype);
        else if (key_dim == 128) launch_ssm<128, 128>(a, n, st, gated_dtype);
        else launch_ssm<256, 128>(a, n, st, gated_dtype);
    } else {
        if (key_dim == 64) launch_ssm<64, 64>(a, n, st, gated_dtype);
        else if (key_dim == 128) launch_ssm<128, 64>(a, n, st, gated_dtype);
        else launch_ssm<256, 64>(a, n, st, gated_dtype);
    }
    return launch_status("ssm_step");
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_rmsnorm_gated(float* out, const float* x, const float* z, const void* w, int w_dtype, long rows,
                                   int heads, int dim, long ld_x, long ld_z, long ld_out, float eps, void* stream) {
    clear_error();
    if (!out || !x || !z || !w) return fail(ANELM_ERR_INVALID, "rmsnorm_gated: null pointer");
    const long span = (long)heads * dim;
    if (rows < 0 || heads <= 0 || dim <= 0 || (rows > 1 && (ld_x < span || ld_z < span || ld_out < span)))
        return fail(ANELM_ERR_INVALID, "rmsnorm_gated: bad sizes or strides");
    if (w_dtype != ANELM_F32 && w_dtype != ANELM_F16 && w_dtype != ANELM_BF16)
        return fail(ANELM_ERR_INVALID, "rmsnorm_gated: weight dtype %d", w_dtype);
    if (rows == 0) return ANELM_OK;
    const dim3 grid(row_blocks(rows * heads));
    hipStream_t st = as_stream(stream);
    if (w_dtype == ANELM_F32)
        hipLaunchKernelGGL((rmsnorm_gated_kernel<ANELM_F32>), grid, dim3(kRowThreads), 0, st, out, x, z, w, rows, heads, dim, ld_x, ld_z, ld_out, eps);
    else if (w_dtype == ANELM_F16)
        hipLaunchKernelGGL((rmsnorm_gated_kernel<ANELM_F16>), grid, dim3(kRowThreads), 0, st, out, x, z, w, rows, heads, dim, ld_x, ld_z, ld_out, eps);
    else
        hipLaunchKernelGGL((rmsnorm_gated_kernel<ANELM_BF16>), grid, dim3(kRowThreads), 0, st, out, x, z, w, rows, heads, dim, ld_x, ld_z, ld_out, eps);
    return launch_status("rmsnorm_gated");
}

extern "C" int anelm_l2_normalize(float* x, long rows, int heads, int dim, long ld, float scale, void* stream) {
    clear_error();
    if (!x) return fail(ANELM_ERR_INVALID, "l2_normalize: null pointer");
    if (rows < 0 || heads <= 0 || dim <= 0 || (rows > 1 && ld < (long)heads * dim))
        return fail(ANELM_ERR_INVALID, "l2_normalize: bad sizes");
    if (rows == 0) return ANELM_OK;
    hipLaunchKernelGGL(l2_normalize_kernel, dim3(row_blocks(rows * heads)), dim3(kRowThreads), 0, as_stream(stream), x,
                       rows, heads, dim, ld, scale);
    return launch_status("l2_normalize");
}

extern "C" int anelm_conv1d_update(float* y, float* conv_state, int32_t* state_pos, const float* x, const float* w,
                                   long batch, int channels, int kernel_size, long ld_x, long ld_y,
                                   long state_stride, void* stream) {
    clear_error();
    if (!y || !conv_state || !state_pos || !x || !w) return fail(ANELM_ERR_INVALID, "conv1d_update: null pointer");
    if (batch < 0 || channels <= 0 || kernel_size < 2)
        return fail(ANELM_ERR_INVALID, "conv1d_update: bad sizes (kernel_size >= 2)");
    if (batch > 1 && (ld_x < channels || ld_y < channels || state_stride < (long)channels * (kernel_size - 1)))
        return fail(ANELM_ERR_INVALID, "conv1d_update: strides overlap");
    if (kernel_size == 4 && !aligned16(w)) return fail(ANELM_ERR_INVALID, "conv1d_update: w not 16-byte aligned");
    if (batch == 0) return ANELM_OK;
    hipLaunchKernelGGL(conv1d_update_kernel, dim3(batch), dim3(1024), 0, as_stream(stream), y, conv_state, state_pos, x,
                       w, channels, kernel_size, ld_x, ld_y, state_stride);
    return launch_status("conv1d_update");
}

extern "C" int anelm_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                              const float* decay, const float* beta, long batch, int n_heads, int n_key_heads,
                              int key_dim, int value_dim, long ld_qk, long ld_v, long ld_y, long state_stride,
                              void* stream) {
    clear_error();
    if (!y || !state || !q || !k || !v || !decay || !beta) return fail(ANELM_ERR_INVALID, "ssm_step: null pointer");
    int rc = ssm_check("ssm_step", batch, n_heads, n_key_heads, key_dim, value_dim, ld_qk, ld_v, ld_y, state_stride,
                       state);
    if (rc) return rc;
    if (batch == 0) return ANELM_OK;
    SsmArgs a{};
    a.y = y; a.state = state; a.q = q; a.k = k; a.v = v; a.decay = decay; a.beta = beta;
    a.nvh = n_heads; a.nkh = n_key_heads; a.ld_qk = ld_qk; a.ld_v = ld_v; a.ld_y = ld_y; a.state_stride = state_stride;
    return ssm_launch(a, batch, n_heads, key_dim, value_dim, -1, as_stream(stream));
}

extern "C" int anelm_ssm_step_gated_norm(float* out, float* state, const float* q, const float* k, const float* v,
                                         const float* decay, const float* beta, const float* z, const void* norm_w,
                                         int w_dtype, long batch, int n_heads, int n_key_heads, int key_dim,
                                         int value_dim, long ld_qk, long ld_v, long ld_z, long ld_out,
                                         long state_stride, float eps, void* stream) {
    clear_error();
    if (!out || !state || !q || !k || !v || !decay || !beta || !z || !norm_w)
        return fail(ANELM_ERR_INVALID, "ssm_step_gated_norm: null pointer");
    if (w_dtype != ANELM_F32 && w_dtype != ANELM_F16 && w_dtype != ANELM_BF16)
        return fail(ANELM_ERR_INVALID, "ssm_step_gated_norm: weight dtype %d", w_dtype);
    int rc = ssm_check("ssm_step_gated_norm", batch, n_heads, n_key_heads, key_dim, value_dim, ld_qk, ld_v, ld_out,
                       state_stride, state);
    if (rc) return rc;
    if (batch > 1 && ld_z < (long)n_heads * value_dim)
        return fail(ANELM_ERR_INVALID, "ssm_step_gated_norm: strides overlap");
    if (batch == 0) return ANELM_OK;
    SsmArgs a{};
    a.state = state; a.q = q; a.k = k; a.v = v; a.decay = decay; a.beta = beta;
    a.nvh = n_heads; a.nkh = n_key_heads; a.ld_qk = ld_qk; a.ld_v = ld_v; a.state_stride = state_stride;
    a.z = z; a.nw = norm_w; a.out = out; a.ld_z = ld_z; a.ld_out = ld_out; a.eps = eps;
    return ssm_launch(a, batch, n_heads, key_dim, value_dim, w_dtype, as_stream(stream));
}

extern "C" int anelm_conv1d_silu_l2norm(float* y, float* conv_state, int32_t* state_pos, const float* x,
                                        const float* w, long batch, int channels, int n_key_heads, long ld_x,
                                        long ld_y, long state_stride, float q_scale, void* stream) {
    clear_error();
    if (!y || !conv_state || !state_pos || !x || !w) return fail(ANELM_ERR_INVALID, "conv1d_silu_l2norm: null pointer");
    if (batch < 0 || channels <= 0 || channels % 128 || n_key_heads < 0 || 2L * n_key_heads * 128 > channels)
        return fail(ANELM_ERR_INVALID, "conv1d_silu_l2norm: channels a multiple of 128 holding 2*n_key_heads heads");
    if (batch > 1 && (ld_x < channels || ld_y < channels || state_stride < (long)channels * 3))
        return fail(ANELM_ERR_INVALID, "conv1d_silu_l2norm: strides overlap");
    if (!aligned16(w)) return fail(ANELM_ERR_INVALID, "conv1d_silu_l2norm: w not 16-byte aligned");
    if (batch == 0) return ANELM_OK;
    const int nblk = channels / 128;
    const int waves = nblk < 16 ? nblk : 16;
    const int bpw = (nblk + waves - 1) / waves;   // blocks per wave: one pass up to 4, more passes past that
    const dim3 grid((unsigned)batch), block((unsigned)(64 * waves));
    hipStream_t st = as_stream(stream);
    const int nq_ch = n_key_heads * 128;
    if (bpw <= 1)
        conv_silu_l2_kernel<1><<<grid, block, 0, st>>>(y, conv_state, state_pos, x, w, channels, nq_ch, ld_x, ld_y,
                                                       state_stride, q_scale);
    else if (bpw == 2)
        conv_silu_l2_kernel<2><<<grid, block, 0, st>>>(y, conv_state, state_pos, x, w, channels, nq_ch, ld_x, ld_y,
                                                       state_stride, q_scale);
    else if (bpw == 3)
        conv_silu_l2_kernel<3><<<grid, block, 0, st>>>(y, conv_state, state_pos, x, w, channels, nq_ch, ld_x, ld_y,
                                                       state_stride, q_scale);
    else
        conv_silu_l2_kernel<4><<<grid, block, 0, st>>>(y, conv_state, state_pos, x, w, channels, nq_ch, ld_x, ld_y,
                                                       state_stride, q_scale);
    return launch_status("conv1d_silu_l2norm");
}

extern "C" int anelm_conv_ssm_step_gated_norm(float* out, float* state, float* conv_state, int32_t* head_pos,
                                              const float* x, const float* conv_w, const float* decay,
                                              const float* beta, const float* z, const void* norm_w, int w_dtype,
                                              long batch, int n_heads, long ld_x, long ld_z, long ld_out,
                                              long state_stride, long conv_state_stride, float q_scale, float eps,
                                              void* stream) {
    const char* fn = "conv_ssm_step_gated_norm";
    clear_error();
    if (!out || !state || !conv_state || !head_pos || !x || !conv_w || !decay || !beta || !z || !norm_w)
        return fail(ANELM_ERR_INVALID, "%s: null pointer", fn);
    if (w_dtype != ANELM_F32 && w_dtype != ANELM_F16 && w_dtype != ANELM_BF16)
        return fail(ANELM_ERR_INVALID, "%s: weight dtype %d", fn, w_dtype);
    if (batch < 0 || n_heads <= 0 || batch > 0x7FFFFFFFL / n_heads)
        return fail(ANELM_ERR_INVALID, "%s: bad sizes", fn);
    const long channels = 3L * n_heads * 128;
    if (batch > 1 && (ld_x < channels || ld_z < (long)n_heads * 128 || ld_out < (long)n_heads * 128 ||
                      state_stride < (long)n_heads * 128 * 128 || conv_state_stride < channels * 3))
        return fail(ANELM_ERR_INVALID, "%s: strides overlap", fn);
    if (!aligned16(state) || (state_stride & 3) || !aligned16(conv_w))
        return fail(ANELM_ERR_INVALID, "%s: state and conv weights 16-byte aligned", fn);
    if (batch == 0) return ANELM_OK;
    ConvSsmArgs a{};
    a.state = state; a.conv_state = conv_state; a.head_pos = head_pos; a.x = x; a.conv_w = conv_w;
    a.decay = decay; a.beta = beta; a.z = z; a.nw = norm_w; a.out = out; a.nh = n_heads;
    a.ld_x = ld_x; a.ld_z = ld_z; a.ld_out = ld_out; a.state_stride = state_stride; a.conv_stride = conv_state_stride;
    a.q_scale = q_scale; a.eps = eps;
    const dim3 grid((unsigned)(batch * n_heads)), block(256);
    hipStream_t st = as_stream(stream);
    if (w_dtype == ANELM_F32) conv_ssm_kernel<ANELM_F32><<<grid, block, 0, st>>>(a);
    else if (w_dtype == ANELM_F16) conv_ssm_kernel<ANELM_F16><<<grid, block, 0, st>>>(a);
    else conv_ssm_kernel<ANELM_BF16><<<grid, block, 0, st>>>(a);
    return launch_status(fn);
}

extern "C" int anelm_matvec(float* y, const float* W, const float* x, long out_dim, int in_dim, void* stream) {
    clear_error();
    if (!y || !W || !x) return fail(ANELM_ERR_INVALID, "matvec: null pointer");
    if (out_dim < 0 || in_dim <= 0) return fail(ANELM_ERR_INVALID, "matvec: bad sizes");
    if (out_dim == 0) return ANELM_OK;
    const dim3 grid(row_blocks(out_dim));
    const bool vec = !(in_dim & 3) && aligned16(W) && aligned16(x);
    if (vec)
        hipLaunchKernelGGL((matvec_kernel<true>), grid, dim3(kRowThreads), 0, as_stream(stream), y, W, x, out_dim, in_dim);
    else
        hipLaunchKernelGGL((matvec_kernel<false>), grid, dim3(kRowThreads), 0, as_stream(stream), y, W, x, out_dim, in_dim);
    return launch_status("matvec");
}
