// The ANE projections with their interface numerics (the conv-as-matvec
// kernels of core/ane_runtime.cpp:265-408, fp16 in and out, :600-640):
//     y[b, o] = fp16(sum_i fp16_rne(x[b, i]) * W16[o, i])   stored as fp32,
// W16 [out_dim, in_dim] row-major fp16 (the truncating convert of the bf16
// checkpoint), fp32 accumulation.  Decode-shaped: a handful to 64 rows of x
// against a weight matrix that is read once, so the kernels are built
// around streaming W at HBM speed, not around reusing it.
//
// MFMA path (in_dim a multiple of 32): v_mfma_f32_16x16x32_f16 with A = a
// 16-row tile of W and B = 16 rows of x (transposed), both fed 8 fp16 per
// lane.  Lane l supplies row (l % 16) of its operand and the 8 inputs
// 8*(l/16) .. +7 of the current 32-input step; D holds output rows
// 4*(l/16) + i (i = 0..3) for batch row l % 16.  A workgroup of 4 waves owns
// 16*RT output rows and 16*NB batch rows; its waves take interleaved 32-input
// steps (so the four read neighbouring 64-byte pieces of each weight row),
// every wave issues the loads of R steps before its first MFMA, and the four
// partial tiles are summed in LDS in a fixed order.  (Splitting the input
// dimension over several workgroups per tile, with the last to finish summing
// the partials behind a device-scope fence, measured 20 us slower per call:
// the fence writes back the L2.)
//
// Dot path (one or two rows of x, up to eight for narrow out_dim; in_dim any
// multiple of 8): one wave per output row, v_dot2_f32_f16 into fp32.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "anelm_common.hpp"

namespace anelm {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float r16(float v) { return (float)to_f16(v); }
// fp16 bits (low 16 of h) widened exactly
__device__ __forceinline__ float h2f_bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__device__ __forceinline__ half8 to_half8(float4 a, float4 b) {
    half8 r;
    r[0] = to_f16(a.x);
    r[1] = to_f16(a.y);
    r[2] = to_f16(a.z);
    r[3] = to_f16(a.w);
    r[4] = to_f16(b.x);
    r[5] = to_f16(b.y);
    r[6] = to_f16(b.z);
    r[7] = to_f16(b.w);
    return r;
}

__device__ __forceinline__ half8 as_half8(uint4 u) {
    half8 r;
    __builtin_memcpy(&r, &u, 16);
    return r;
}

// (x * s) * gamma for four inputs, gamma as two packed bf16 pairs: the fused
// RMSNorm's output, before its fp16 rounding
__device__ __forceinline__ float4 norm_scale(float4 v, float s, uint32_t g01, uint32_t g23) {
    v.x = (v.x * s) * bf16_to_f32(g01 & 0xFFFFu);
    v.y = (v.y * s) * bf16_to_f32(g01 >> 16);
    v.z = (v.z * s) * bf16_to_f32(g23 & 0xFFFFu);
    v.w = (v.w * s) * bf16_to_f32(g23 >> 16);
    return v;
}

struct ProjArgs {
    float* y;
    const void* x;  // fp32, or fp16 already rounded (XH)
    const uint16_t* w;
    int out_dim, in_dim, batch;
    long ld_x, ld_y;
    // fused prologue (kNorm): x replaced by rmsnorm(x) * gamma, gamma bf16 [in_dim]
    const uint16_t* gamma;
    float eps;
    // SwiGLU epilogue (kSwiGLU, kSwiGLU16): the up rows follow the gate rows at this offset
    long pair_rows;
    // kSwiGLU16, kStore16: the output as fp16 bits (row stride ld_y) instead of y
    uint16_t* y16;
    // y rows 16-byte aligned (y and ld_y), for the LDS kernel's float4 stores
    bool vec_y;
};

// What the epilogue does with the rounded projection p = fp16(sum) (as fp32):
enum Epilogue {
    kStore = 0,   // y = p
    kAdd = 1,     // y = y + p  (the residual add of qwen3.cpp:516, :527)
    kSwiGLU = 2,  // y = silu(p_gate) * p_up  (core/ane_runtime.cpp:393-395)
    kSwiGLU16 = 3,  // the same rounded to fp16 (nearest even) into y16: the next projection's input
    kStore16 = 4,   // y16 = p as fp16 bits (the ANE kernels' own fp16 output)
    kSwiGLU16T = 5, // kSwiGLU16 with y16 in the tiled layout (out_dim columns): the tiled projection's input
};
constexpr bool is_swiglu(int epi) { return epi == kSwiGLU || epi == kSwiGLU16 || epi == kSwiGLU16T; }

// kNorm (fp32 x): the workgroup first computes the RMSNorm scale
// 1/sqrtf(ss/dim + eps) of each of its batch rows (core/cpu_ops.cpp:25-31),
// and every input is formed as (x * s) * gamma before its fp16 rounding,
// exactly the separate RMSNorm's output.  kSwiGLU needs RT = 2: tile 0 holds
// gate rows, tile 1 the up rows pair_rows further on, and out_dim counts the
// gate rows.
// TILED: W in the tiled layout of anelm_proj_tile_f16 (the 16 x 32 block of
// a row tile and an input step as one contiguous 1 KB piece in lane order),
// so a weight load instruction reads 1 KB in a row rather than 64 bytes from
// each of 16 rows a row pitch apart, which lands on few L2 channels.  XT:
// the fp16 x in the same layout (batch rows as its rows).  The operands, and
// so the outputs, are the same as with row-major W and x.
template <bool XH, int NB, int RT, int R, bool NORM = false, int EPI = kStore, int NW = 4, bool TILED = false,
          bool XT = false>
__global__ __launch_bounds__(64 * NW) void proj_mfma_kernel(ProjArgs a) {
    static_assert(!XT || XH, "the tiled x is fp16");
    static_assert(!NORM || !XH, "the fused norm reads fp32 x");
    static_assert(!is_swiglu(EPI) || RT == 2, "SwiGLU pairs a gate tile with an up tile");
    __shared__ float4v part[NW][RT * NB][64];
    __shared__ float s_scale[16 * NB];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const long row0 = (long)blockIdx.x * 16 * (is_swiglu(EPI) ? 1 : RT);
    const int b0 = blockIdx.y * 16 * NB;
    // operand rows, clamped: rows past the end compute values that are never
    // stored (TILED: tiles past the last load the last one; the SwiGLU's up
    // tiles start pair_rows/16 tiles on, pair_rows a multiple of 16)
    const uint16_t* wp[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        if constexpr (TILED) {
            const long ntile = (a.out_dim + 15) / 16;
            long tile = row0 / 16 + (is_swiglu(EPI) ? 0 : t);
            tile = tile < ntile ? tile : ntile - 1;
            if (is_swiglu(EPI) && t == 1) tile += a.pair_rows / 16;
            wp[t] = a.w + (tile * (a.in_dim / 32) * 64 + lane) * 8;
        } else {
            const long r0 = is_swiglu(EPI) ? row0 + c : row0 + 16 * t + c;
            const long r = (r0 < a.out_dim ? r0 : a.out_dim - 1) + (is_swiglu(EPI) && t == 1 ? a.pair_rows : 0);
            wp[t] = a.w + r * a.in_dim + 8 * g;
        }
    }
    // x rows (clamped); XT: the batch tile's pieces (tiles past the last load the last one)
    long xoff[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        if constexpr (XT) {
            const long bt = b0 / 16 + nb, last = (a.batch - 1) / 16;
            xoff[nb] = ((bt < last ? bt : last) * (a.in_dim / 32) * 64 + lane) * 8;
        } else {
            const int b = b0 + nb * 16 + c;
            xoff[nb] = (long)(b < a.batch ? b : a.batch - 1) * a.ld_x + 8 * g;
        }
    }
    const float* xf = static_cast<const float*>(a.x);
    const uint16_t* xh = static_cast<const uint16_t*>(a.x);
    const int s_end = a.in_dim / 32;  // 32-input steps

    // the loads of R steps of this wave, starting at step s0
    uint4 wr[R][RT];
    float4 xr[R][XH ? 1 : NB][2];
    uint4 xq[R][XH ? NB : 1];
    uint4 gq[NORM ? R : 1];
    auto issue = [&](int s0) {
#pragma unroll
        for (int j = 0; j < R; j++) {
            const int s = s0 + NW * j;
            const int k = 32 * (s < s_end ? s : s_end - 1);  // clamped: in bounds, result unused
#pragma unroll
            for (int t = 0; t < RT; t++) wr[j][t] = ld_nt(reinterpret_cast<const uint4*>(wp[t] + (TILED ? 16L * k : k)));
            if constexpr (NORM) gq[j] = *reinterpret_cast<const uint4*>(a.gamma + k + 8 * g);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                if constexpr (XH) {
                    xq[j][nb] = *reinterpret_cast<const uint4*>(xh + xoff[nb] + (XT ? 16L * k : k));
                } else {
                    xr[j][nb][0] = *reinterpret_cast<const float4*>(xf + xoff[nb] + k);
                    xr[j][nb][1] = *reinterpret_cast<const float4*>(xf + xoff[nb] + k + 4);
                }
            }
        }
    };
    // the first round's loads go out before the RMSNorm prologue, whose own
    // loads then overlap them
    issue(wv);
    // the residual add's y values are loaded now, with the weights, not after
    // the reduction (addresses clamped: lanes without an output load a valid
    // element and never use it)
    constexpr int QPW = (RT * NB + NW - 1) / NW;  // epilogue tiles per wave
    float yprev[EPI == kAdd ? QPW : 1][4];
    if constexpr (EPI == kAdd) {
#pragma unroll
        for (int j = 0; j < QPW; j++) {
            const int q = wv + j * NW < RT * NB ? wv + j * NW : RT * NB - 1;
            const int b = b0 + (q % NB) * 16 + c;
            const float* yr = a.y + (long)(b < a.batch ? b : a.batch - 1) * a.ld_y;
            const long r = row0 + 16 * (q / NB) + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; i++) yprev[j][i] = yr[r + i < a.out_dim ? r + i : a.out_dim - 1];
        }
    }

    if constexpr (NORM) {
        // wave w: the workgroup's batch rows w, w+NW, ... that exist; each
        // lane has four 16-byte loads in flight per round (a 1024-wide row in one)
        const int nrows = a.batch - b0 < 16 * NB ? a.batch - b0 : 16 * NB;
        if ((int)threadIdx.x < 16 * NB && (int)threadIdx.x >= nrows) s_scale[threadIdx.x] = 0.0f;  // unused columns
        for (int i = wv; i < nrows; i += NW) {
            const float* xrow = xf + (long)(b0 + i) * a.ld_x;
            float sp[4] = {0.f, 0.f, 0.f, 0.f};
            for (int k = 4 * lane; k < a.in_dim; k += 1024) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++)
                    v[u] = k + 256 * u < a.in_dim ? *reinterpret_cast<const float4*>(xrow + k + 256 * u)
                                                  : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    sp[u] = fmaf(v[u].x, v[u].x, sp[u]);
                    sp[u] = fmaf(v[u].y, v[u].y, sp[u]);
                    sp[u] = fmaf(v[u].z, v[u].z, sp[u]);
                    sp[u] = fmaf(v[u].w, v[u].w, sp[u]);
                }
            }
            const float ss = wave_sum((sp[0] + sp[1]) + (sp[2] + sp[3]));
            if (lane == 0) s_scale[i] = 1.0f / sqrtf(ss / (float)a.in_dim + a.eps);
        }
        __syncthreads();
    }
    float my_scale[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) my_scale[nb] = NORM ? s_scale[16 * nb + c] : 1.0f;

    float4v acc[RT][NB];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) acc[t][nb] = float4v{0.f, 0.f, 0.f, 0.f};
    for (int s0 = wv; s0 < s_end; s0 += NW * R) {
        if (s0 != wv) issue(s0);
#pragma unroll
        for (int j = 0; j < R; j++) {
            if (s0 + NW * j < s_end) {  // wave-uniform
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    half8 xb;
                    if constexpr (XH) {
                        xb = as_half8(xq[j][nb]);
                    } else if constexpr (NORM) {
                        const float4 u = xr[j][nb][0], v = xr[j][nb][1];
                        const uint4 q = gq[j];
                        xb = to_half8(norm_scale(u, my_scale[nb], q.x, q.y), norm_scale(v, my_scale[nb], q.z, q.w));
                    } else {
                        xb = to_half8(xr[j][nb][0], xr[j][nb][1]);
                    }
#pragma unroll
                    for (int t = 0; t < RT; t++)
                        acc[t][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(wr[j][t]), xb, acc[t][nb], 0, 0, 0);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) part[wv][t * NB + nb][lane] = acc[t][nb];
    __syncthreads();
    if constexpr (is_swiglu(EPI)) {
        for (int nb = wv; nb < NB; nb += NW) {
            float4v gs = part[0][nb][lane], us = part[0][NB + nb][lane];
            for (int w = 1; w < NW; w++) {
                gs += part[w][nb][lane];
                us += part[w][NB + nb][lane];
            }
            const int b = b0 + nb * 16 + c;
            const long r = row0 + 4 * g;
            if (b < a.batch) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (r + i < a.out_dim) {
                        const float h = silu_ref(r16(gs[i])) * r16(us[i]);
                        if constexpr (EPI == kSwiGLU16)
                            a.y16[(long)b * a.ld_y + r + i] = __builtin_bit_cast(uint16_t, to_f16(h));
                        else if constexpr (EPI == kSwiGLU16T)
                            a.y16[tiled_index(b, (int)(r + i), a.out_dim)] = __builtin_bit_cast(uint16_t, to_f16(h));
                        else
                            a.y[(long)b * a.ld_y + r + i] = h;
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < QPW; j++) {
            const int q = wv + j * NW;
            if (q >= RT * NB) break;
            float4v s = part[0][q][lane];
            for (int w = 1; w < NW; w++) s += part[w][q][lane];
            const int t = q / NB, nb = q % NB;
            const int b = b0 + nb * 16 + c;
            const long r = row0 + 16 * t + 4 * g;
            if (b < a.batch) {
                float* yr = a.y + (long)b * a.ld_y;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (r + i < a.out_dim) {
                        if constexpr (EPI == kAdd) yr[r + i] = yprev[j][i] + r16(s[i]);
                        else if constexpr (EPI == kStore16)
                            a.y16[(long)b * a.ld_y + r + i] = __builtin_bit_cast(uint16_t, to_f16(s[i]));
                        else yr[r + i] = r16(s[i]);
                    }
                }
            }
        }
    }
}

// ---- many rows of x against a long W: x staged in LDS ------------------------
// The LM head past 16 sequences (151936 output rows): every weight row must
// be read from HBM once while each serves all the batch rows.  A workgroup
// stages 16*NB rows of the fp16 x in LDS once (rows padded by 16 bytes, so
// the 16 rows a ds_read_b128 of a wave touches fall in 16 different bank
// groups).  Its 8 waves then take 8 adjacent 16-row tiles of W (128 output
// rows) per round, rounds striding over the grid (about one workgroup per
// CU, so W streams once), each wave streaming its tile over the full input
// dimension: 8 steps of 32 inputs per load chunk, the next chunk's loads in
// flight during the current chunk's MFMAs, each 16-byte weight load feeding
// NB MFMAs with x from LDS.  At a round's end the waves round their sums to
// fp16 into an LDS staging block, and the workgroup stores the 128 outputs
// of each batch row as one contiguous run (fp32 widened, non-temporal, or
// fp16 bits with kStore16): stored straight from the MFMA layout, each batch
// row got 64-byte pieces, which cost a third of the kernel's time.  Weight
// loads are cached (non-temporal measured slower here).  in_dim a multiple
// of 256.
// TILED: W in the tiled layout of anelm_proj_tile_f16, where the 16 bytes
// that lane l loads for a 16-row tile and a 32-input step lie at lane l's
// place in one contiguous 1 KB block, so every weight load instruction reads
// 1 KB in a row instead of 64 bytes from each of 16 rows.  The MFMA operands
// are the same values either way, so are the outputs.
constexpr int kLdsR = 8;                       // 32-input steps per load chunk
constexpr int kLdsHalves = 64 * (1024 + 8);    // the LDS x area: 64 rows of 1024 inputs, or fewer longer rows
constexpr int kYsLd = 128 + 8;                 // staging row stride (fp16), 128 outputs per batch row

__host__ __device__ constexpr int lds_rows(int in_dim) {   // batch rows staged per workgroup
    return 64 * (in_dim + 8) <= kLdsHalves ? 64 : (32 * (in_dim + 8) <= kLdsHalves ? 32 : 16);
}

template <int NB, int EPI, bool TILED = false>
__global__ __launch_bounds__(512) void proj_lds_kernel(ProjArgs a) {
    static_assert(EPI == kStore || EPI == kStore16, "store epilogues only");
    __shared__ __align__(16) uint16_t xs[kLdsHalves];
    __shared__ __align__(16) uint16_t ys[16 * NB * kYsLd];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int K = a.in_dim, ldx = K + 8;
    const int b0 = blockIdx.y * 16 * NB;
    const uint16_t* xh = static_cast<const uint16_t*>(a.x);
    const int ngroup = (a.out_dim + 127) / 128;   // 128-row groups (8 tiles)
    const int rounds = (ngroup - 1 - (int)blockIdx.x) / (int)gridDim.x + 1;
    const int cpt = K / (32 * kLdsR);             // load chunks per tile
    const int nq = rounds * cpt;                  // every wave runs all of them (barriers)
    const uint16_t* wbase = a.w + 8 * (lane >> 4);
    // the R loads of chunk q (clamped rows: tiles past the end load a valid
    // row, computed and never stored; a chunk past nq reloads the last one)
    auto issue = [&](uint4* w, int q) {
        q = q < nq ? q : nq - 1;
        const int grp = (int)blockIdx.x + (q / cpt) * (int)gridDim.x;
        if constexpr (TILED) {
            // tile 8*grp + wv (clamped to the last; rows past out_dim are zeros)
            const long ntile = (a.out_dim + 15) / 16;
            long t = 8L * grp + wv;
            t = t < ntile ? t : ntile - 1;
            const uint16_t* p = a.w + ((t * (K / 32) + (q % cpt) * kLdsR) * 64 + lane) * 8;
#pragma unroll
            for (int j = 0; j < kLdsR; j++) w[j] = *reinterpret_cast<const uint4*>(p + 512 * j);
        } else {
            long r = 128L * grp + 16 * wv + (lane & 15);
            r = r < a.out_dim ? r : a.out_dim - 1;
            const uint16_t* p = wbase + r * K + (q % cpt) * (32 * kLdsR);
#pragma unroll
            for (int j = 0; j < kLdsR; j++) w[j] = *reinterpret_cast<const uint4*>(p + 32 * j);
        }
    };
    if ((int)blockIdx.x >= ngroup) return;        // whole workgroup (before any barrier)
    // the first weight chunk does not depend on x: its loads go out before
    // the x staging, so the two latencies overlap
    uint4 wa[kLdsR], wb[kLdsR];
    issue(wa, 0);
    __builtin_amdgcn_sched_barrier(0);
    {   // stage x rows b0 .. b0 + 16*NB - 1 (zeros past the batch): 8 loads per lane before their stores
        const int qpr = K / 8, nx = 16 * NB * qpr;
        for (int base = 0; base < nx; base += 8 * (int)blockDim.x) {
            uint4 t[8];
            int dst[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int idx = base + u * (int)blockDim.x + (int)threadIdx.x;
                const int ic = idx < nx ? idx : nx - 1;   // past the end: the last quad again
                const int r = ic / qpr, c = ic - r * qpr;
                const int b = b0 + r < a.batch ? b0 + r : a.batch - 1;
                t[u] = *reinterpret_cast<const uint4*>(xh + (long)b * a.ld_x + 8 * c);
                if (b0 + r >= a.batch) t[u] = make_uint4(0u, 0u, 0u, 0u);
                dst[u] = r * ldx + 8 * c;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) *reinterpret_cast<uint4*>(xs + dst[u]) = t[u];
        }
    }
    __syncthreads();
    const uint16_t* xrow = xs + (lane & 15) * ldx + 8 * (lane >> 4);
    float4v acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) acc[nb] = float4v{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const uint4* w, int q) {
        const int s0 = (q % cpt) * kLdsR;
#pragma unroll
        for (int j = 0; j < kLdsR; j++) {
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                const uint4 xq = *reinterpret_cast<const uint4*>(xrow + nb * 16 * ldx + 32 * (s0 + j));
                acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(w[j]), as_half8(xq), acc[nb], 0, 0, 0);
            }
        }
        if (q % cpt == cpt - 1) {   // the round is complete (workgroup-uniform)
            // lane: outputs 16*wv + 4*(lane/16) + i of batch row nb*16 + lane%16
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                uint16_t h[4];
#pragma unroll
                for (int i = 0; i < 4; i++) h[i] = __builtin_bit_cast(uint16_t, to_f16(acc[nb][i]));
                *reinterpret_cast<uint2*>(ys + (nb * 16 + (lane & 15)) * kYsLd + 16 * wv + 4 * (lane >> 4)) =
                    make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
                acc[nb] = float4v{0.f, 0.f, 0.f, 0.f};
            }
            __syncthreads();
            // 16*NB batch rows x 32 quads of 4 outputs, 512 lanes
            const long c0 = 128L * ((int)blockIdx.x + (q / cpt) * (int)gridDim.x);
#pragma unroll
            for (int u = 0; u < NB; u++) {
                const int item = u * 512 + (int)threadIdx.x;
                const int br = item >> 5, c4 = item & 31;
                const int b = b0 + br;
                const long col = c0 + 4 * c4;
                const uint2 hv = *reinterpret_cast<const uint2*>(ys + br * kYsLd + 4 * c4);
                if (b < a.batch) {
                    if constexpr (EPI == kStore16) {
                        uint16_t* yr = a.y16 + (long)b * a.ld_y;
                        if (col + 3 < a.out_dim && a.vec_y) {
                            *reinterpret_cast<uint2*>(yr + col) = hv;
                        } else {
                            const uint16_t e[4] = {(uint16_t)(hv.x & 0xFFFFu), (uint16_t)(hv.x >> 16),
                                                   (uint16_t)(hv.y & 0xFFFFu), (uint16_t)(hv.y >> 16)};
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                if (col + i < a.out_dim) yr[col + i] = e[i];
                        }
                    } else {
                        float* yr = a.y + (long)b * a.ld_y;
                        const float4 f = make_float4(h2f_bits(hv.x & 0xFFFFu), h2f_bits(hv.x >> 16),
                                                     h2f_bits(hv.y & 0xFFFFu), h2f_bits(hv.y >> 16));
                        if (col + 3 < a.out_dim && a.vec_y) {
                            st_nt(reinterpret_cast<float4*>(yr + col), f);   // 67.7 against 73.8 us cached
                        } else {
                            const float e[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                if (col + i < a.out_dim) yr[col + i] = e[i];
                        }
                    }
                }
            }
            __syncthreads();   // the staging block is reused next round
        }
    };
    // The scheduling barriers keep each chunk's loads ahead of the previous
    // chunk's MFMAs; without them the scheduler sank the loads below the
    // MFMAs, leaving one chunk in flight.
    // Both chunks of an iteration are computed; an odd last chunk (already
    // in wa) is computed after the loop.  With a conditional second compute
    // inside the loop, the back edge merged a path with wb's loads still in
    // flight, and the compiler put a vmcnt wait at the loop head (after a
    // round's stores it waited on half of the chunk just issued).
    int q = 0;
    for (; q + 1 < nq; q += 2) {
        issue(wb, q + 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(wa, q);
        __builtin_amdgcn_sched_barrier(0);
        issue(wa, q + 2);
        __builtin_amdgcn_sched_barrier(0);
        compute(wb, q + 1);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (q < nq) compute(wa, q);
}

// ---- one or two rows of x: one wave per output row ------------------------
// Below a few rows of x the 16-column MFMA tile is mostly idle and the work
// is a matrix-vector product bound by how fast W streams in.  Here each wave
// owns RPW output rows (2*RPW with the SwiGLU's up rows) for BT rows of x;
// lane l covers inputs 8l .. 8l+7 of every 512-input chunk, one 16-byte load
// of each weight row, and the loads of NCH chunks are in flight together.
// Products are v_dot2_f32_f16 of fp16 pairs into fp32 (a fp16 x fp16
// product is exact in fp32), a wave sum closes each row, and lane t of the
// wave writes row t's result.  Small out_dim gets the most from it: 1024
// output rows are 64 MFMA workgroups but 1024 waves here.
//
// x comes in one of three forms (XM), each giving the same fp16 operand the
// MFMA path uses:
//   kXF32   fp32 rows, rounded to fp16 per element on the way in;
//   kXNorm  fp32 rows through the fused RMSNorm: the workgroup loads each row
//           once, reduces its sum of squares and writes the normalised row,
//           rounded to fp16, to LDS, where the waves read it (one 16-byte
//           read per chunk instead of two 16-byte global loads and a gamma
//           load);
//   kXF16   fp16 rows already rounded by their producer (the attention's
//           fp16 output, the SwiGLU's fp16 store): half the bytes of fp32.
// At the one-sequence decode shapes the activation loads were as many
// instructions as the weight loads or more (fp32 x: two 16-byte loads per
// one of W), and taking them out of the loop saved 0.5-1.1 us of 3.7-5.2 us.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2v as_half2(uint32_t u) {
    half2v r;
    __builtin_memcpy(&r, &u, 4);
    return r;
}

__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, to_f16(lo)) | ((uint32_t)__builtin_bit_cast(uint16_t, to_f16(hi)) << 16);
}

enum : int {
    kXF32 = 0,
    kXNorm = 1,
    kXF16 = 2,
};
constexpr int kDotNormMaxIn = 4096;   // kXNorm: LDS for the staged rows (8 KB per row of x)

// kXNorm: 4-input slices per thread that cover in_dim for a chunk count
constexpr int dot_norm_slices(int nch) { return nch <= 2 ? 1 : (nch <= 4 ? 2 : 4); }

template <int BT, int RPW, int NCH, int XM, int EPI>
__global__ __launch_bounds__(256) void proj_dot_kernel(ProjArgs a) {
    constexpr int NR = is_swiglu(EPI) ? 2 * RPW : RPW;  // weight rows per wave
    constexpr bool NORM = XM == kXNorm;
    constexpr int NS = dot_norm_slices(NCH);
    __shared__ float s_part[4][BT];
    __shared__ uint4 s_x16[NORM ? BT : 1][NORM ? kDotNormMaxIn / 8 : 1];   // 8 fp16 inputs per entry
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const long r0 = ((long)blockIdx.x * 4 + wv) * RPW;
    // operand rows, clamped: rows past the end compute values that are never stored
    const uint16_t* wp[NR];
#pragma unroll
    for (int t = 0; t < NR; t++) {
        const long r = r0 + t % RPW;
        wp[t] = a.w + ((r < a.out_dim ? r : a.out_dim - 1) + (t >= RPW ? a.pair_rows : 0)) * a.in_dim;
    }
    const float* xf = static_cast<const float*>(a.x);
    const uint16_t* xh = static_cast<const uint16_t*>(a.x);
    uint4 wr[NCH][NR];
    int idx[NCH];  // this lane's first input in each chunk, clamped into the row
    auto issue = [&](int c0) {
#pragma unroll
        for (int k = 0; k < NCH; k++) {
            const int i = c0 + 512 * k + 8 * lane;
            idx[k] = i < a.in_dim ? i : a.in_dim - 8;
#pragma unroll
            for (int t = 0; t < NR; t++) wr[k][t] = ld_nt(reinterpret_cast<const uint4*>(wp[t] + idx[k]));
        }
    };
    // kXNorm: thread j's slices of x, inputs 4j + 1024s .. +3 (in_dim <=
    // 1024*NS, a multiple of 8), and their gammas.  They are loaded before the
    // first weight chunks: loads retire in issue order, so the prologue
    // below waits only for these while the weights are still in flight.
    // Rows past the batch and inputs past in_dim are zeros, which leave the
    // sums unchanged and stage as zeros.
    float4 xs[NORM ? BT : 1][NORM ? NS : 1];
    uint2 gs[NORM ? NS : 1];
    if constexpr (NORM) {
#pragma unroll
        for (int sl = 0; sl < NS; sl++) {
            const int k = 4 * (int)threadIdx.x + 1024 * sl;
            gs[sl] = k < a.in_dim ? *reinterpret_cast<const uint2*>(a.gamma + k) : make_uint2(0u, 0u);
#pragma unroll
            for (int b = 0; b < BT; b++)
                xs[b][sl] = k < a.in_dim && b < a.batch ? *reinterpret_cast<const float4*>(xf + (long)b * a.ld_x + k)
                                                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // the first chunks' weight loads, and the residual add's y value with
    // them (lane b*RPW + t: row r0 + t of x row b; clamped, unused where the
    // lane stores nothing)
    issue(0);
    float yprev = 0.f;
    if constexpr (EPI == kAdd) {
        const int t = lane % RPW, b = lane / RPW < a.batch ? lane / RPW : a.batch - 1;
        const long r = r0 + t < a.out_dim ? r0 + t : a.out_dim - 1;
        yprev = a.y[(long)b * a.ld_y + r];
    }

    if constexpr (NORM) {
        // the workgroup's 256 lanes share each row's sum of squares
#pragma unroll
        for (int b = 0; b < BT; b++) {
            float sp = 0.f;
#pragma unroll
            for (int sl = 0; sl < NS; sl++) {
                sp = fmaf(xs[b][sl].x, xs[b][sl].x, sp);
                sp = fmaf(xs[b][sl].y, xs[b][sl].y, sp);
                sp = fmaf(xs[b][sl].z, xs[b][sl].z, sp);
                sp = fmaf(xs[b][sl].w, xs[b][sl].w, sp);
            }
            sp = wave_sum_rows(sp);
            if (lane == 0) s_part[wv][b] = sp;
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < BT; b++) {
            const float ss = (s_part[0][b] + s_part[1][b]) + (s_part[2][b] + s_part[3][b]);
            const float scale = 1.0f / sqrtf(ss / (float)a.in_dim + a.eps);
            uint16_t* row = reinterpret_cast<uint16_t*>(&s_x16[b][0]);
#pragma unroll
            for (int sl = 0; sl < NS; sl++) {
                const int k = 4 * (int)threadIdx.x + 1024 * sl;
                if (k < a.in_dim) {
                    const float4 v = norm_scale(xs[b][sl], scale, gs[sl].x, gs[sl].y);
                    *reinterpret_cast<uint2*>(row + k) = make_uint2(pack_f16(v.x, v.y), pack_f16(v.z, v.w));
                }
            }
        }
        __syncthreads();
    }
    if (r0 >= a.out_dim) return;  // whole wave, after the workgroup's barriers

    float acc[NR][BT];
#pragma unroll
    for (int t = 0; t < NR; t++)
#pragma unroll
        for (int b = 0; b < BT; b++) acc[t][b] = 0.f;
    for (int c0 = 0; c0 < a.in_dim; c0 += 512 * NCH) {
        if (c0) issue(c0);
#pragma unroll
        for (int k = 0; k < NCH; k++) {
            const bool live = c0 + 512 * k + 8 * lane < a.in_dim;
#pragma unroll
            for (int b = 0; b < BT; b++) {
                const int bb = b < a.batch ? b : a.batch - 1;
                half2v x0, x1, x2, x3;
                if constexpr (XM == kXF32) {
                    const float* xp = xf + (long)bb * a.ld_x + idx[k];
                    const float4 p = reinterpret_cast<const float4*>(xp)[0];
                    const float4 q = reinterpret_cast<const float4*>(xp)[1];
                    const _Float16 z = (_Float16)0.0f;
                    x0 = live ? half2v{to_f16(p.x), to_f16(p.y)} : half2v{z, z};
                    x1 = live ? half2v{to_f16(p.z), to_f16(p.w)} : half2v{z, z};
                    x2 = live ? half2v{to_f16(q.x), to_f16(q.y)} : half2v{z, z};
                    x3 = live ? half2v{to_f16(q.z), to_f16(q.w)} : half2v{z, z};
                } else {
                    uint4 xv;
                    if constexpr (NORM) xv = s_x16[b][idx[k] >> 3];
                    else xv = *reinterpret_cast<const uint4*>(xh + (long)bb * a.ld_x + idx[k]);
                    if (!live) xv = make_uint4(0u, 0u, 0u, 0u);
                    x0 = as_half2(xv.x);
                    x1 = as_half2(xv.y);
                    x2 = as_half2(xv.z);
                    x3 = as_half2(xv.w);
                }
#pragma unroll
                for (int t = 0; t < NR; t++) {
                    float s = acc[t][b];
                    s = __builtin_amdgcn_fdot2(as_half2(wr[k][t].x), x0, s, false);
                    s = __builtin_amdgcn_fdot2(as_half2(wr[k][t].y), x1, s, false);
                    s = __builtin_amdgcn_fdot2(as_half2(wr[k][t].z), x2, s, false);
                    s = __builtin_amdgcn_fdot2(as_half2(wr[k][t].w), x3, s, false);
                    acc[t][b] = s;
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NR; t++)
#pragma unroll
        for (int b = 0; b < BT; b++) acc[t][b] = wave_sum_rows(acc[t][b]);
    // lane b*RPW + t stores row r0 + t of x row b
    float s = 0.f, u = 0.f;
#pragma unroll
    for (int t = 0; t < RPW; t++)
#pragma unroll
        for (int b = 0; b < BT; b++)
            if (lane == b * RPW + t) {
                s = acc[t][b];
                if constexpr (is_swiglu(EPI)) u = acc[RPW + t][b];
            }
    const int t = lane % RPW, b = lane / RPW;
    if (lane < RPW * BT && b < a.batch && r0 + t < a.out_dim) {
        const long o = (long)b * a.ld_y + r0 + t;
        if constexpr (EPI == kAdd) a.y[o] = yprev + r16(s);
        else if constexpr (EPI == kSwiGLU) a.y[o] = silu_ref(r16(s)) * r16(u);
        else if constexpr (EPI == kSwiGLU16) a.y16[o] = __builtin_bit_cast(uint16_t, to_f16(silu_ref(r16(s)) * r16(u)));
        else if constexpr (EPI == kStore16) a.y16[o] = __builtin_bit_cast(uint16_t, to_f16(s));
        else a.y[o] = r16(s);
    }
}

template <int BT, int RPW, int NCH, int XM, int EPI>
void launch_dot(const ProjArgs& a, hipStream_t st) {
    const long waves = (a.out_dim + RPW - 1) / RPW;
    proj_dot_kernel<BT, RPW, NCH, XM, EPI><<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st>>>(a);
}

// Launch shape: all of a 1024-input row in one round of loads (NCH = 2),
// longer rows in rounds of up to six 512-input chunks; two output rows per
// wave from 4096 rows up and four from 32768 (the LM head), so that each
// wave has several loads in flight, one row per wave for the SwiGLU's row
// pairs and for narrow out_dim, so that there are enough waves.
template <int BT, int XM, int EPI>
void dot_shape(const ProjArgs& a, hipStream_t st) {
    const int chunks = (a.in_dim + 511) / 512;
    if (chunks > 2) {
        if (chunks <= 4) launch_dot<BT, 1, 4, XM, EPI>(a, st);
        else launch_dot<BT, 1, 6, XM, EPI>(a, st);
        return;
    }
    if constexpr (!is_swiglu(EPI)) {
        if constexpr (BT == 1) {
            if (a.out_dim >= 32768) return launch_dot<1, 4, 2, XM, EPI>(a, st);
        }
        if (a.out_dim >= 4096) return launch_dot<BT, 2, 2, XM, EPI>(a, st);
    }
    launch_dot<BT, 1, 2, XM, EPI>(a, st);
}

template <int XM, int EPI>
void proj_dot(const ProjArgs& a, hipStream_t st) {
    if (a.batch == 1) dot_shape<1, XM, EPI>(a, st);
    else if (a.batch == 2) dot_shape<2, XM, EPI>(a, st);
    else if (a.batch <= 4) dot_shape<4, XM, EPI>(a, st);
    else dot_shape<8, XM, EPI>(a, st);
}

// Where the dot kernel beats the MFMA kernel (measured at the Qwen3-0.6B
// decode shapes): one or two rows of x everywhere, up to eight for narrow
// out_dim (1024 rows: 64 MFMA workgroups).
bool dot_wins(long batch, int out_dim) { return batch <= 2 || (batch <= 8 && out_dim <= 1024); }

// y and x must not share memory: workgroups write y while others still read x.
bool overlaps(const void* y, long ld_y, int out_dim, int y_bytes, const void* x, long ld_x, int in_dim, int x_bytes,
              long batch) {
    const uintptr_t y0 = reinterpret_cast<uintptr_t>(y), x0 = reinterpret_cast<uintptr_t>(x);
    const uintptr_t y1 = y0 + (uintptr_t)((batch - 1) * ld_y + out_dim) * (uintptr_t)y_bytes;
    const uintptr_t x1 = x0 + (uintptr_t)((batch - 1) * ld_x + in_dim) * (uintptr_t)x_bytes;
    return x0 < y1 && y0 < x1;
}

// Whether [p, p + np) and [q, q + nq) (bytes) share a byte.
bool spans_overlap(const void* p, long np, const void* q, long nq) {
    const uintptr_t p0 = reinterpret_cast<uintptr_t>(p), q0 = reinterpret_cast<uintptr_t>(q);
    return p0 < q0 + (uintptr_t)nq && q0 < p0 + (uintptr_t)np;
}

bool dot_ok(const float* x, const uint16_t* w16, long batch, int in_dim, long ld_x) {
    return batch <= 8 && in_dim % 8 == 0 && ld_x % 4 == 0 && aligned16(x) && aligned16(w16);
}
// fp16 rows: one 16-byte load per 8 inputs
bool dot16_ok(const uint16_t* x16, const uint16_t* w16, long batch, int in_dim, long ld_x) {
    return batch <= 8 && in_dim % 8 == 0 && ld_x % 8 == 0 && aligned16(x16) && aligned16(w16);
}

// ---- any shape (the fallback) ------------------------------------------------
// One wave per (batch row, output row): lanes stride over the inputs, fp16
// products (exact in fp32) accumulated in fp32, a wave sum, one rounding to
// fp16.  For shapes the kernels above do not take (in_dim not a multiple of
// 8, unaligned rows); it reads x once per output row, so it is slow on large
// shapes, which no Qwen3 size produces.
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <bool XH, int EPI>
__global__ __launch_bounds__(256) void proj_generic_kernel(ProjArgs a) {
    static_assert(EPI == kStore || EPI == kStore16, "store epilogues only");
    const int lane = threadIdx.x & 63;
    const long gwave = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const long o = gwave % a.out_dim, b = gwave / a.out_dim;
    if (b >= a.batch) return;   // whole wave
    const uint16_t* wr = a.w + o * a.in_dim;
    const float* xf = static_cast<const float*>(a.x) + b * a.ld_x;
    const uint16_t* xh = static_cast<const uint16_t*>(a.x) + b * a.ld_x;
    float s = 0.f;
    for (int i = lane; i < a.in_dim; i += 64) s = fmaf(XH ? h2f(xh[i]) : r16(xf[i]), h2f(wr[i]), s);
    s = wave_sum(s);
    if (lane == 0) {
        if constexpr (EPI == kStore16) a.y16[b * a.ld_y + o] = __builtin_bit_cast(uint16_t, to_f16(s));
        else a.y[b * a.ld_y + o] = r16(s);
    }
}

template <bool XH, int EPI>
void launch_generic(const ProjArgs& a, hipStream_t st) {
    const long waves = (long)a.out_dim * a.batch;
    proj_generic_kernel<XH, EPI><<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st>>>(a);
}

// ---- the LDS kernel's launch -----------------------------------------------------
// compute units of the current device (cached per device)
int cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Past 16 rows of fp16 x, against at least 8192 output rows: W streams once
// through the LDS kernel (measured for the 151936-row LM head; narrower W is
// better served by more, smaller workgroups).
bool lds_ok(const ProjArgs& a) {
    return a.batch > 16 && a.out_dim >= 8192 && a.in_dim % 256 == 0 && a.in_dim <= 4096 && a.ld_x % 8 == 0 &&
           aligned16(a.x) && aligned16(a.w);
}

template <int EPI, bool TILED = false>
void launch_lds(ProjArgs a, hipStream_t st) {
    const int rows = lds_rows(a.in_dim);
    const int ngroup = (a.out_dim + 127) / 128;
    const int gx = std::min(cu_count(), ngroup);
    const dim3 grid((unsigned)gx, (unsigned)((a.batch + rows - 1) / rows));
    a.vec_y = EPI == kStore ? aligned16(a.y) && a.ld_y % 4 == 0 : aligned8(a.y16) && a.ld_y % 4 == 0;
    if (rows == 64) proj_lds_kernel<4, EPI, TILED><<<grid, dim3(512), 0, st>>>(a);
    else if (rows == 32) proj_lds_kernel<2, EPI, TILED><<<grid, dim3(512), 0, st>>>(a);
    else proj_lds_kernel<1, EPI, TILED><<<grid, dim3(512), 0, st>>>(a);
}

// The tiled layout: for 16-row tile t and 32-input step s, 64 pieces of 16
// bytes (8 fp16), piece l = W[16t + l%16][32s + 8(l/16) .. +7], the block at
// ((t * in_dim/32 + s) * 64) pieces; rows past out_dim are zeros.  One
// thread per piece.
__global__ __launch_bounds__(256) void tile_w16_kernel(uint16_t* dst, const uint16_t* src, int out_dim, int in_dim,
                                                       long npieces) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= npieces) return;
    const int steps = in_dim / 32;
    const int l = (int)(i & 63);
    const long ts = i >> 6;
    const int st = (int)(ts % steps);
    const long t = ts / steps;
    const long r = 16 * t + (l & 15);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (r < out_dim) v = *reinterpret_cast<const uint4*>(src + r * in_dim + 32 * st + 8 * (l >> 4));
    *reinterpret_cast<uint4*>(dst + 8 * i) = v;
}

// ---- MFMA launch shapes -----------------------------------------------------
template <bool XH, int NB, int RT, int R, bool NORM = false, int EPI = kStore, int NW = 4, bool TILED = false,
          bool XT = false>
void launch_mfma(const ProjArgs& a, hipStream_t st) {
    const int rows = 16 * (is_swiglu(EPI) ? 1 : RT);
    const dim3 grid((unsigned)((a.out_dim + rows - 1) / rows), (unsigned)((a.batch + 16 * NB - 1) / (16 * NB)));
    proj_mfma_kernel<XH, NB, RT, R, NORM, EPI, NW, TILED, XT><<<grid, dim3(64 * NW), 0, st>>>(a);
}

// Up to 16 rows: one 16-row batch block, one row tile per workgroup (the
// most workgroups), 8 steps of loads in flight per wave.  Past 16 rows,
// 32-row batch blocks with two row tiles per workgroup (each input fetched
// from cache feeds four MFMA tiles) where that still leaves enough
// workgroups; shapes with few output tiles (out_dim 1024 at 64 rows: 64 such
// workgroups) keep 16x16 tiles and four times the workgroups, which measured
// 1.6x faster there.  (8 waves per workgroup for the few-tile shapes
// measured 10% slower than 4.)
template <bool XH>
int proj_mfma(const ProjArgs& a, hipStream_t st) {
    const long tiles16 = (long)((a.out_dim + 15) / 16) * ((a.batch + 15) / 16);
    if (XH && lds_ok(a)) launch_lds<kStore>(a, st);
    else if (a.batch <= 16 || tiles16 < 512) launch_mfma<XH, 1, 1, 8>(a, st);
    else launch_mfma<XH, 2, 2, XH ? 8 : 4>(a, st);
    return launch_status("proj_f16");
}

bool mfma_ok(const void* x, bool x_f16, const uint16_t* w16, int in_dim, long ld_x) {
    return in_dim % 32 == 0 && aligned16(x) && aligned16(w16) && ld_x % (x_f16 ? 8 : 4) == 0;
}

bool sizes_ok(long batch, int out_dim, int in_dim, long ld_x, long ld_y) {
    return batch > 0 && batch <= 65535 * 32L && out_dim > 0 && in_dim > 0 && ld_x >= in_dim && ld_y >= out_dim &&
           (long)out_dim * in_dim <= (1L << 40);
}

ProjArgs args(float* y, const void* x, const uint16_t* w16, long batch, int out_dim, int in_dim, long ld_x,
              long ld_y) {
    ProjArgs a = {};
    a.y = y;
    a.x = x;
    a.w = w16;
    a.out_dim = out_dim;
    a.in_dim = in_dim;
    a.batch = (int)batch;
    a.ld_x = ld_x;
    a.ld_y = ld_y;
    return a;
}

}  // namespace

}  // namespace anelm

using namespace anelm;

// fp32 in, fp32 out (holding fp16 values): the whole fp16 projection,
// conversions included, with each weight read once.
extern "C" int anelm_proj_f16(float* y, const float* x, const uint16_t* w16, long batch, int out_dim, int in_dim,
                              long ld_x, long ld_y, void* stream) {
    clear_error();
    if (!y || !x || !w16) return fail(ANELM_ERR_INVALID, "proj_f16: null pointer");
    if (!sizes_ok(batch, out_dim, in_dim, ld_x, ld_y)) return fail(ANELM_ERR_INVALID, "proj_f16: bad sizes or strides");
    if (overlaps(y, ld_y, out_dim, 4, x, ld_x, in_dim, 4, batch))
        return fail(ANELM_ERR_INVALID, "proj_f16: y overlaps x (y is written while x is still read)");
    hipStream_t st = as_stream(stream);
    const ProjArgs a = args(y, x, w16, batch, out_dim, in_dim, ld_x, ld_y);
    const bool dot = dot_ok(x, w16, batch, in_dim, ld_x);
    if (mfma_ok(x, false, w16, in_dim, ld_x) && !(dot && dot_wins(batch, out_dim))) return proj_mfma<false>(a, st);
    if (dot) {
        proj_dot<kXF32, kStore>(a, st);
    } else {
        if ((long)out_dim * batch > (1L << 33)) return fail(ANELM_ERR_INVALID, "proj_f16: too large for its shape");
        launch_generic<false, kStore>(a, st);
    }
    return launch_status("proj_f16");
}

// The same with x already rounded to fp16 (e.g. by anelm_f32_to_f16): for
// larger batches, where rounding x once beats rounding it in every workgroup.
extern "C" int anelm_proj_f16_x16(float* y, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim,
                                  int in_dim, long ld_x, long ld_y, void* stream) {
    clear_error();
    if (!y || !x16 || !w16) return fail(ANELM_ERR_INVALID, "proj_f16_x16: null pointer");
    if (!sizes_ok(batch, out_dim, in_dim, ld_x, ld_y))
        return fail(ANELM_ERR_INVALID, "proj_f16_x16: bad sizes or strides");
    if (overlaps(y, ld_y, out_dim, 4, x16, ld_x, in_dim, 2, batch))
        return fail(ANELM_ERR_INVALID, "proj_f16_x16: y overlaps x (y is written while x is still read)");
    if (!mfma_ok(x16, true, w16, in_dim, ld_x))
        return fail(ANELM_ERR_INVALID,
                    "proj_f16_x16: needs in_dim a multiple of 32, ld_x a multiple of 8, 16-byte aligned x and W");
    return proj_mfma<true>(args(y, x16, w16, batch, out_dim, in_dim, ld_x, ld_y), as_stream(stream));
}

// fp32 inputs with the fused RMSNorm and epilogues: one 16-row batch block
// per workgroup up to 16 rows, and past that wherever there are few output
// tiles; otherwise 32-row batch blocks and two row tiles per workgroup.
template <bool NORM, int EPI>
void f32_fused(const ProjArgs& a, hipStream_t st) {
    const long tiles16 = (long)((a.out_dim + 15) / 16) * ((a.batch + 15) / 16);
    constexpr int RT = is_swiglu(EPI) ? 2 : 1;
    if (a.batch <= 16 || (!is_swiglu(EPI) && tiles16 < 512)) launch_mfma<false, 1, RT, 8, NORM, EPI>(a, st);
    else launch_mfma<false, 2, 2, 4, NORM, EPI>(a, st);
}

// The fused epilogues on fp16 inputs (x16 from anelm_rmsnorm_f16 or a
// previous fp16 SwiGLU): the decode step past a few rows, where the fp32
// inputs' extra bytes and per-workgroup rounding cost more than the
// separate conversion.
// The SwiGLU past 32 rows takes all 64 batch rows of a workgroup (each
// gate|up tile read by one workgroup): 9.8 us against 11.8 us with 32 at the
// Qwen3-0.6B shape and 64 rows; the other shapes measured no better so.
// Shapes on fp16 x (every one 4 waves splitting the input steps, so every
// shape gives the same bits).  Up to 16 rows: one 16-row batch block, one row
// tile per workgroup, 8 steps of loads in flight per wave.  Past 16 rows
// (measured at 64 rows on the Qwen3-0.6B layer shapes): the SwiGLU's gate|up
// tile pairs take all 64 batch rows of a workgroup with 8 steps in flight;
// shapes with many output tiles take 32 x 32 tiles; the others 16 x 16 tiles
// with a wave's whole share of the input steps (up to 24) in flight at once.
template <int EPI, bool TILED = false, bool XT = false>
void x16_mfma(const ProjArgs& a, hipStream_t st) {
    const long tiles16 = (long)((a.out_dim + 15) / 16) * ((a.batch + 15) / 16);
    constexpr int RT = is_swiglu(EPI) ? 2 : 1;
    const int steps = a.in_dim / 32 / 4;   // per wave
    if (a.batch <= 16) {
        launch_mfma<true, 1, RT, 8, false, EPI, 4, TILED, XT>(a, st);
    } else if constexpr (is_swiglu(EPI)) {
        if (a.batch > 32) launch_mfma<true, 4, 2, 8, false, EPI, 4, TILED, XT>(a, st);
        else launch_mfma<true, 2, 2, 8, false, EPI, 4, TILED, XT>(a, st);
    } else {
        if (tiles16 >= 512) launch_mfma<true, 2, 2, 8, false, EPI, 4, TILED, XT>(a, st);
        else if (steps > 16) launch_mfma<true, 1, 1, 24, false, EPI, 4, TILED, XT>(a, st);
        else if (steps > 8) launch_mfma<true, 1, 1, 16, false, EPI, 4, TILED, XT>(a, st);
        else launch_mfma<true, 1, 1, 8, false, EPI, 4, TILED, XT>(a, st);
    }
}

template <int EPI>
void x16_fused(const ProjArgs& a, hipStream_t st) {
    if (dot16_ok(static_cast<const uint16_t*>(a.x), a.w, a.batch, a.in_dim, a.ld_x) && dot_wins(a.batch, a.out_dim))
        proj_dot<kXF16, EPI>(a, st);
    else if (EPI == kStore && lds_ok(a)) launch_lds<kStore>(a, st);
    else x16_mfma<EPI>(a, st);
}

extern "C" int anelm_proj_f16_x16_fused(void* y, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim,
                                        int in_dim, long ld_x, long ld_y, int epilogue, void* stream) {
    clear_error();
    if (!y || !x16 || !w16) return fail(ANELM_ERR_INVALID, "proj_f16_x16_fused: null pointer");
    if (!sizes_ok(batch, out_dim, in_dim, ld_x, ld_y))
        return fail(ANELM_ERR_INVALID, "proj_f16_x16_fused: bad sizes or strides");
    if (!mfma_ok(x16, true, w16, in_dim, ld_x))
        return fail(ANELM_ERR_INVALID,
                    "proj_f16_x16_fused: needs in_dim a multiple of 32, ld_x a multiple of 8, 16-byte aligned x and W");
    if (epilogue < ANELM_PROJ_STORE || epilogue > ANELM_PROJ_SWIGLU_F16)
        return fail(ANELM_ERR_INVALID, "proj_f16_x16_fused: unknown epilogue %d", epilogue);
    if (overlaps(y, ld_y, out_dim, epilogue == ANELM_PROJ_SWIGLU_F16 ? 2 : 4, x16, ld_x, in_dim, 2, batch))
        return fail(ANELM_ERR_INVALID, "proj_f16_x16_fused: y overlaps x (y is written while x is still read)");
    ProjArgs a = args(static_cast<float*>(y), x16, w16, batch, out_dim, in_dim, ld_x, ld_y);
    a.y16 = static_cast<uint16_t*>(y);
    a.pair_rows = out_dim;
    hipStream_t st = as_stream(stream);
    switch (epilogue) {
        case ANELM_PROJ_STORE: x16_fused<kStore>(a, st); break;
        case ANELM_PROJ_ADD: x16_fused<kAdd>(a, st); break;
        case ANELM_PROJ_SWIGLU: x16_fused<kSwiGLU>(a, st); break;
        default: x16_fused<kSwiGLU16>(a, st); break;
    }
    return launch_status("proj_f16_x16_fused");
}

extern "C" size_t anelm_proj_tiled_size(int out_dim, int in_dim) {
    if (out_dim <= 0 || in_dim <= 0 || in_dim % 32 != 0) return 0;
    return (size_t)((out_dim + 15) / 16) * 16 * (size_t)in_dim * sizeof(uint16_t);
}

extern "C" int anelm_proj_tile_f16(uint16_t* w_tiled, const uint16_t* w16, int out_dim, int in_dim, void* stream) {
    clear_error();
    if (!w_tiled || !w16) return fail(ANELM_ERR_INVALID, "proj_tile_f16: null pointer");
    if (out_dim <= 0 || in_dim <= 0 || in_dim % 32 != 0 || (long)out_dim * in_dim > (1L << 40))
        return fail(ANELM_ERR_INVALID, "proj_tile_f16: out_dim %d, in_dim %d (a multiple of 32)", out_dim, in_dim);
    if (!aligned16(w_tiled) || !aligned16(w16)) return fail(ANELM_ERR_INVALID, "proj_tile_f16: needs 16-byte alignment");
    const size_t bytes = anelm_proj_tiled_size(out_dim, in_dim);
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(w_tiled), s0 = reinterpret_cast<uintptr_t>(w16);
    if (d0 < s0 + (uintptr_t)out_dim * in_dim * 2 && s0 < d0 + bytes)
        return fail(ANELM_ERR_INVALID, "proj_tile_f16: the tiled copy overlaps W");
    const long npieces = (long)(bytes / 16);
    tile_w16_kernel<<<dim3((unsigned)((npieces + 255) / 256)), dim3(256), 0, as_stream(stream)>>>(w_tiled, w16, out_dim,
                                                                                                 in_dim, npieces);
    return launch_status("proj_tile_f16");
}

extern "C" int anelm_proj_f16_x16_tiled(void* y, const uint16_t* x16, const uint16_t* w_tiled, long batch, int out_dim,
                                        int in_dim, long ld_x, long ld_y, int epilogue, void* stream) {
    clear_error();
    if (!y || !x16 || !w_tiled) return fail(ANELM_ERR_INVALID, "proj_f16_x16_tiled: null pointer");
    if (!sizes_ok(batch, out_dim, in_dim, ld_x, ld_y))
        return fail(ANELM_ERR_INVALID, "proj_f16_x16_tiled: bad sizes or strides");
    if (in_dim % 32 != 0 || ld_x % 8 != 0 || !aligned16(x16) || !aligned16(w_tiled))
        return fail(ANELM_ERR_INVALID,
                    "proj_f16_x16_tiled: needs in_dim a multiple of 32, ld_x a multiple of 8, 16-byte aligned x and W");
    if (epilogue < ANELM_PROJ_STORE || epilogue > ANELM_PROJ_STORE_F16)
        return fail(ANELM_ERR_INVALID, "proj_f16_x16_tiled: unknown epilogue %d", epilogue);
    const bool swiglu = epilogue == ANELM_PROJ_SWIGLU || epilogue == ANELM_PROJ_SWIGLU_F16;
    if (swiglu && out_dim % 16 != 0)
        return fail(ANELM_ERR_INVALID, "proj_f16_x16_tiled: the SwiGLU needs out_dim (gate rows) a multiple of 16");
    const bool f16 = epilogue == ANELM_PROJ_STORE_F16 || epilogue == ANELM_PROJ_SWIGLU_F16;
    if (overlaps(y, ld_y, out_dim, f16 ? 2 : 4, x16, ld_x, in_dim, 2, batch))
        return fail(ANELM_ERR_INVALID, "proj_f16_x16_tiled: y overlaps x (y is written while x is still read)");
    ProjArgs a = args(static_cast<float*>(y), x16, w_tiled, batch, out_dim, in_dim, ld_x, ld_y);
    a.y16 = static_cast<uint16_t*>(y);
    a.pair_rows = out_dim;
    hipStream_t st = as_stream(stream);
    // the stores stream W through the LDS kernel where anelm_proj_f16_x16_fused
    // does (past 16 rows, at least 8192 output rows) and up to 16 rows; the
    // rest takes the MFMA kernel's shapes of anelm_proj_f16_x16_fused
    const bool lds_shape = in_dim % 256 == 0 && in_dim <= 4096;
    const bool store = epilogue == ANELM_PROJ_STORE || epilogue == ANELM_PROJ_STORE_F16;
    if (store && lds_shape && (batch <= 16 || lds_ok(a))) {
        if (f16) launch_lds<kStore16, true>(a, st);
        else launch_lds<kStore, true>(a, st);
        return launch_status("proj_f16_x16_tiled");
    }
    switch (epilogue) {
        case ANELM_PROJ_STORE: x16_mfma<kStore, true>(a, st); break;
        case ANELM_PROJ_ADD: x16_mfma<kAdd, true>(a, st); break;
        case ANELM_PROJ_SWIGLU: x16_mfma<kSwiGLU, true>(a, st); break;
        case ANELM_PROJ_SWIGLU_F16: x16_mfma<kSwiGLU16, true>(a, st); break;
        default: x16_mfma<kStore16, true>(a, st); break;
    }
    return launch_status("proj_f16_x16_tiled");
}

extern "C" int anelm_proj_f16_tt(void* y, const uint16_t* x_t, const uint16_t* w_t, long batch, int out_dim,
                                 int in_dim, long ld_y, int epilogue, void* stream) {
    clear_error();
    const char* fn = "proj_f16_tt";
    if (!y || !x_t || !w_t) return fail(ANELM_ERR_INVALID, "%s: null pointer", fn);
    if (!sizes_ok(batch, out_dim, in_dim, in_dim, ld_y) || in_dim % 32 != 0)
        return fail(ANELM_ERR_INVALID, "%s: bad sizes or strides (in_dim a multiple of 32)", fn);
    if (!aligned16(x_t) || !aligned16(w_t)) return fail(ANELM_ERR_INVALID, "%s: needs 16-byte aligned x and W", fn);
    if (epilogue < ANELM_PROJ_STORE || epilogue > ANELM_PROJ_SWIGLU_F16_TILED)
        return fail(ANELM_ERR_INVALID, "%s: unknown epilogue %d", fn, epilogue);
    const bool swiglu = epilogue == ANELM_PROJ_SWIGLU || epilogue == ANELM_PROJ_SWIGLU_F16 ||
                        epilogue == ANELM_PROJ_SWIGLU_F16_TILED;
    if (swiglu && out_dim % 16 != 0)
        return fail(ANELM_ERR_INVALID, "%s: the SwiGLU needs out_dim (gate rows) a multiple of 16", fn);
    if (epilogue == ANELM_PROJ_SWIGLU_F16_TILED && (out_dim % 32 != 0 || !aligned16(y)))
        return fail(ANELM_ERR_INVALID, "%s: the tiled output needs out_dim a multiple of 32 and 16-byte alignment", fn);
    // x_t holds ceil(batch/16)*16 rows; y its rows (or, tiled, as many padded rows)
    const long xrows = (batch + 15) / 16 * 16;
    const int ybytes = epilogue == ANELM_PROJ_STORE_F16 || epilogue == ANELM_PROJ_SWIGLU_F16 ? 2 : 4;
    const bool ytiled = epilogue == ANELM_PROJ_SWIGLU_F16_TILED;
    // y spans its batch rows (tiled: the padded rows), x_t its padded rows
    if (spans_overlap(y, ytiled ? xrows * out_dim * 2 : ((batch - 1) * ld_y + out_dim) * ybytes, x_t,
                      xrows * in_dim * 2))
        return fail(ANELM_ERR_INVALID, "%s: y overlaps x (y is written while x is still read)", fn);
    ProjArgs a = args(static_cast<float*>(y), x_t, w_t, batch, out_dim, in_dim, in_dim, ytiled ? out_dim : ld_y);
    a.y16 = static_cast<uint16_t*>(y);
    a.pair_rows = out_dim;
    hipStream_t st = as_stream(stream);
    switch (epilogue) {
        case ANELM_PROJ_STORE: x16_mfma<kStore, true, true>(a, st); break;
        case ANELM_PROJ_ADD: x16_mfma<kAdd, true, true>(a, st); break;
        case ANELM_PROJ_SWIGLU: x16_mfma<kSwiGLU, true, true>(a, st); break;
        case ANELM_PROJ_SWIGLU_F16: x16_mfma<kSwiGLU16, true, true>(a, st); break;
        case ANELM_PROJ_STORE_F16: x16_mfma<kStore16, true, true>(a, st); break;
        default: x16_mfma<kSwiGLU16T, true, true>(a, st); break;
    }
    return launch_status(fn);
}

// Decode-step projections with the neighbouring layer ops fused in, for up
// to 16 rows (see the header): the RMSNorm before a projection, the residual
// add after one, the SwiGLU between the gate|up and down projections.
extern "C" int anelm_proj_f16_fused(void* y, const float* x, const uint16_t* w16, long batch, int out_dim,
                                    int in_dim, long ld_x, long ld_y, const uint16_t* norm_bf16, float eps,
                                    int epilogue, void* stream) {
    clear_error();
    if (!y || !x || !w16) return fail(ANELM_ERR_INVALID, "proj_f16_fused: null pointer");
    if (!sizes_ok(batch, out_dim, in_dim, ld_x, ld_y))
        return fail(ANELM_ERR_INVALID, "proj_f16_fused: bad sizes or strides");
    if (!mfma_ok(x, false, w16, in_dim, ld_x) || (norm_bf16 && !aligned16(norm_bf16)))
        return fail(ANELM_ERR_INVALID,
                    "proj_f16_fused: needs in_dim a multiple of 32, ld_x a multiple of 4, 16-byte aligned x, W, gamma");
    if (epilogue < ANELM_PROJ_STORE || epilogue > ANELM_PROJ_SWIGLU_F16)
        return fail(ANELM_ERR_INVALID, "proj_f16_fused: unknown epilogue %d", epilogue);
    if (overlaps(y, ld_y, out_dim, epilogue == ANELM_PROJ_SWIGLU_F16 ? 2 : 4, x, ld_x, in_dim, 4, batch))
        return fail(ANELM_ERR_INVALID,
                    "proj_f16_fused: y overlaps x (y is written while x is still read; the residual add takes the "
                    "residual stream as y and the projection input as a separate x)");
    ProjArgs a = args(static_cast<float*>(y), x, w16, batch, out_dim, in_dim, ld_x, ld_y);
    a.y16 = static_cast<uint16_t*>(y);
    a.gamma = norm_bf16;
    a.eps = eps;
    a.pair_rows = out_dim;  // SwiGLU: W holds out_dim gate rows, then out_dim up rows
    hipStream_t st = as_stream(stream);
    const bool norm = norm_bf16 != nullptr;
    if (dot_ok(x, w16, batch, in_dim, ld_x) && dot_wins(batch, out_dim) && (!norm || in_dim <= kDotNormMaxIn)) {
        switch (epilogue) {
            case ANELM_PROJ_STORE:
                if (norm) proj_dot<kXNorm, kStore>(a, st);
                else proj_dot<kXF32, kStore>(a, st);
                break;
            case ANELM_PROJ_ADD:
                if (norm) proj_dot<kXNorm, kAdd>(a, st);
                else proj_dot<kXF32, kAdd>(a, st);
                break;
            case ANELM_PROJ_SWIGLU:
                if (norm) proj_dot<kXNorm, kSwiGLU>(a, st);
                else proj_dot<kXF32, kSwiGLU>(a, st);
                break;
            default:
                if (norm) proj_dot<kXNorm, kSwiGLU16>(a, st);
                else proj_dot<kXF32, kSwiGLU16>(a, st);
                break;
        }
        return launch_status("proj_f16_fused");
    }
    switch (epilogue) {
        case ANELM_PROJ_STORE:
            if (norm) f32_fused<true, kStore>(a, st);
            else f32_fused<false, kStore>(a, st);
            break;
        case ANELM_PROJ_ADD:
            if (norm) f32_fused<true, kAdd>(a, st);
            else f32_fused<false, kAdd>(a, st);
            break;
        case ANELM_PROJ_SWIGLU:
            if (norm) f32_fused<true, kSwiGLU>(a, st);
            else f32_fused<false, kSwiGLU>(a, st);
            break;
        default:
            if (norm) f32_fused<true, kSwiGLU16>(a, st);
            else f32_fused<false, kSwiGLU16>(a, st);
            break;
    }
    return launch_status("proj_f16_fused");
}

// The ANE projection with fp16 rows in and out: y16 = fp16(x16 . W16^T),
// fp32 accumulation, one rounding to nearest even.
extern "C" int anelm_linear_f16(uint16_t* y16, const uint16_t* x16, const uint16_t* w16, long batch, int out_dim,
                                int in_dim, long ld_x, long ld_y, void* stream) {
    clear_error();
    if (!y16 || !x16 || !w16) return fail(ANELM_ERR_INVALID, "linear_f16: null pointer");
    if (!sizes_ok(batch, out_dim, in_dim, ld_x, ld_y) || (long)out_dim * batch > (1L << 33))
        return fail(ANELM_ERR_INVALID, "linear_f16: bad sizes or strides");
    if (overlaps(y16, ld_y, out_dim, 2, x16, ld_x, in_dim, 2, batch))
        return fail(ANELM_ERR_INVALID, "linear_f16: y overlaps x (y is written while x is still read)");
    ProjArgs a = args(nullptr, x16, w16, batch, out_dim, in_dim, ld_x, ld_y);
    a.y16 = y16;
    hipStream_t st = as_stream(stream);
    if (lds_ok(a)) launch_lds<kStore16>(a, st);
    else if (mfma_ok(x16, true, w16, in_dim, ld_x)) launch_mfma<true, 1, 1, 8, false, kStore16>(a, st);
    else launch_generic<true, kStore16>(a, st);
    return launch_status("linear_f16");
}
