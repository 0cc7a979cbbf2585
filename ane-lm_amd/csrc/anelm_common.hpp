// Shared device helpers and host-side argument / launch checking for the
// gfx950 fused layer-op kernels.  Wave size is 64 (CDNA); every kernel is
// written for it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "anelm_hip.h"

namespace anelm {

constexpr int kWave = 64;

// ------------------------------------------------------------ host side

// Records a formatted message as this thread's last error and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears this thread's last error.
void clear_error();
// Maps the state after a launch to a status (ANELM_ERR_HIP on a launch error).
int launch_status(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Up to 512 inverse frequencies passed to kernels by value.
struct InvFreq {
    float v[512];
};
// inv[j] = 1.0f / powf(theta, (float)(2j) / (float)rot_dim), evaluated on the
// host with the C library exactly as models/llm/qwen3.cpp:206-209 does, so
// device angles pos*inv[j] are bit-identical to the reference's.
void rope_inv_freq(InvFreq* out, int rot_dim, float theta);

// ------------------------------------------------------------ device side

__device__ __forceinline__ float wave_sum(float v) {
    v += __shfl_xor(v, 32);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 1);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 32));
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 8));
    v = fmaxf(v, __shfl_xor(v, 4));
    v = fmaxf(v, __shfl_xor(v, 2));
    v = fmaxf(v, __shfl_xor(v, 1));
    return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of 16 lanes (a DPP row), every lane of the group
// active; each step adds a lane's value to its partner's, which holds the
// same bits, so all 16 lanes end with the same sum.
__device__ __forceinline__ float group16_sum(float v) {
    v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);   // row_half_mirror: the other quad of the half row
    v += dpp_f32<0x140>(v);   // row_mirror: the other half row
    return v;
}

// Sum over the wave, every lane receiving it: the 16-lane DPP sums, then
// the four row sums (lanes 0, 16, 32, 48) added in a fixed order.  DPP moves
// and lane reads take a few cycles each, where each step of a shuffle sum
// (wave_sum) is an LDS permute round trip.  Every lane of the wave active.
__device__ __forceinline__ float wave_sum_rows(float v) {
    v = group16_sum(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Maximum over the wave, every lane receiving it, the same way (fmaxf).
__device__ __forceinline__ float wave_max_rows(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp_f32<0x140>(v));   // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Element (r, c) of an fp16 matrix with `cols` columns (a multiple of 32)
// in the tiled layout of anelm_proj_tile_f16: for each 16-row tile and
// 32-column step, the 16 x 32 block as 64 pieces of 8, piece l holding row
// 16t + l%16, columns 32s + 8(l/16) .. +7.
__device__ __forceinline__ long tiled_index(long r, int c, int cols) {
    return (((r >> 4) * (cols >> 5) + (c >> 5)) * 64 + (r & 15) + 16 * ((c & 31) >> 3)) * 8 + (c & 7);
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
        lo = __shfl_xor(lo, d);
        hi = __shfl_xor(hi, d);
        v += ((uint64_t)hi << 32) | lo;
    }
    return v;
}

// Exact fp16 -> fp32 widening with the reference's conventions
// (include/ane_lm/common.h:35-56): subnormals m * 2^-24 (exact), exponent 31
// keeps the mantissa bits (NaN payload preserved, no quieting).
__device__ __forceinline__ float f16_to_f32_exact(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t normal = sign | ((e + 112u) << 23) | (m << 13);
    uint32_t special = sign | 0x7F800000u | (m << 13);
    uint32_t sub = sign | __float_as_uint((float)m * 0x1p-24f);
    return __uint_as_float(e == 0 ? sub : (e == 31 ? special : normal));
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// The reference's truncating bf16 -> fp16 (include/ane_lm/common.h:58-75) on
// the low 16 bits of b, in integer arithmetic only.
__device__ __forceinline__ uint32_t bf16_to_f16_trunc(uint32_t b) {
    uint32_t sign = b & 0x8000u;
    int e = (int)((b >> 7) & 0xFFu) - 112;        // fp16 exponent field
    uint32_t m = (b & 0x7Fu) << 16;               // fp32 mantissa field
    uint32_t normal = sign | ((uint32_t)e << 10) | (m >> 13);
    int sh = 1 - e;                               // 1..11 on the subnormal branch
    sh = sh < 0 ? 0 : (sh > 31 ? 31 : sh);
    uint32_t sub = sign | (((m | 0x800000u) >> sh) >> 13);
    uint32_t r = e >= 31 ? (sign | 0x7C00u) : (e > 0 ? normal : (e < -10 ? sign : sub));
    return r;
}

// Weight element i as fp32 for the three storage types (fp16/bf16 widening
// is exact).
template <int DT>
__device__ __forceinline__ float load_w(const void* w, long i);
template <>
__device__ __forceinline__ float load_w<ANELM_F32>(const void* w, long i) {
    return static_cast<const float*>(w)[i];
}
template <>
__device__ __forceinline__ float load_w<ANELM_F16>(const void* w, long i) {
    return f16_to_f32_exact(static_cast<const uint16_t*>(w)[i]);
}
template <>
__device__ __forceinline__ float load_w<ANELM_BF16>(const void* w, long i) {
    return bf16_to_f32(static_cast<const uint16_t*>(w)[i]);
}

// Four consecutive weights starting at i (i % 4 == 0, w 16/8-byte aligned).
template <int DT>
__device__ __forceinline__ float4 load_w4(const void* w, long i);
template <>
__device__ __forceinline__ float4 load_w4<ANELM_F32>(const void* w, long i) {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(w) + i);
}
template <>
__device__ __forceinline__ float4 load_w4<ANELM_F16>(const void* w, long i) {
    uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + i);
    return make_float4(f16_to_f32_exact(v.x & 0xFFFFu), f16_to_f32_exact(v.x >> 16),
                       f16_to_f32_exact(v.y & 0xFFFFu), f16_to_f32_exact(v.y >> 16));
}
template <>
__device__ __forceinline__ float4 load_w4<ANELM_BF16>(const void* w, long i) {
    uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + i);
    return make_float4(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16),
                       bf16_to_f32(v.y & 0xFFFFu), bf16_to_f32(v.y >> 16));
}

// core/cpu_ops.cpp:7-14 form: silu(g) = g / (1 + expf(-g)) with a correctly
// rounded divide.  Shared by the SwiGLU kernel and the projection epilogue
// that fuses it, so both give the same bits.
__device__ __forceinline__ float silu_ref(float g) {
    const float t = expf(-g) + 1.0f;
    return g / t;
}

// One KV ring step for a sequence's state (start, len), models/llm/qwen3.cpp
// :475-488, with the state clamped into range first (0 <= len <= cap, start
// mod cap): while len < cap the row goes to slot start+len (mod cap) and len
// grows, afterwards it overwrites slot start and start advances.  Returns the
// slot and stores the advanced state.
__device__ __forceinline__ int ring_advance(int32_t* rs, int32_t* rl, int cap) {
    int s = *rs, l = *rl;
    l = l < 0 ? 0 : (l > cap ? cap : l);
    s %= cap;
    if (s < 0) s += cap;
    int slot;
    if (l < cap) {
        slot = s + l;
        if (slot >= cap) slot -= cap;
        l++;
    } else {
        slot = s;
        s++;
        if (s >= cap) s = 0;
    }
    *rs = s;
    *rl = l;
    return slot;
}

// fp32 -> fp16 rounded to nearest even, of the value as already rounded to
// fp32.  Without the empty asm the compiler folds a preceding multiply or
// add into v_fma_mixlo_f16, which rounds the exact result once, straight to
// fp16 (it does so even under -ffp-contract=off), so a product such as
// (x * s) * gamma could land one fp16 ulp away from the reference's fp32
// result rounded to fp16.
__device__ __forceinline__ _Float16 to_f16(float v) {
    __asm__("" : "+v"(v));
    return (_Float16)v;
}

// Non-temporal 16-byte loads / stores (streamed data that is touched once).
typedef float nat_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int nat_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_nt(const float4* p) {
    const nat_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nat_f32x4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float4* p, float4 v) {
    const nat_f32x4 n = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(n, reinterpret_cast<nat_f32x4*>(p));
}
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
    const nat_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nat_u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(uint4* p, uint4 v) {
    const nat_u32x4 n = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(n, reinterpret_cast<nat_u32x4*>(p));
}

// This lane's four gammas as raw storage bits, fetched with the row (for
// fp32 gammas the float4 itself); widened after the reduction.
template <int DT>
struct Gamma4 {
    uint2 bits;
    __device__ __forceinline__ void load(const void* w, int c) {
        bits = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + c);
    }
    // fp16: the conversion instruction widens every non-NaN value exactly
    // (normal, subnormal, zero, infinity) in one operation; a NaN keeps its
    // payload unquieted only through the integer widening, which the wave
    // takes when any of its lanes holds one.
    __device__ __forceinline__ float4 get() const {
        if constexpr (DT == ANELM_F16) {
            const float4 f = make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(bits.x & 0xFFFFu)),
                                         (float)__builtin_bit_cast(_Float16, (uint16_t)(bits.x >> 16)),
                                         (float)__builtin_bit_cast(_Float16, (uint16_t)(bits.y & 0xFFFFu)),
                                         (float)__builtin_bit_cast(_Float16, (uint16_t)(bits.y >> 16)));
            const bool nan = f.x != f.x || f.y != f.y || f.z != f.z || f.w != f.w;
            if (__builtin_expect(__ballot(nan) != 0, 0))
                return make_float4(f16_to_f32_exact(bits.x & 0xFFFFu), f16_to_f32_exact(bits.x >> 16),
                                   f16_to_f32_exact(bits.y & 0xFFFFu), f16_to_f32_exact(bits.y >> 16));
            return f;
        } else
            return make_float4(bf16_to_f32(bits.x & 0xFFFFu), bf16_to_f32(bits.x >> 16), bf16_to_f32(bits.y & 0xFFFFu),
                               bf16_to_f32(bits.y >> 16));
    }
};
template <>
struct Gamma4<ANELM_F32> {
    float4 v;
    __device__ __forceinline__ void load(const void* w, int c) { v = *reinterpret_cast<const float4*>(static_cast<const float*>(w) + c); }
    __device__ __forceinline__ float4 get() const { return v; }
};

// Launch geometry of the row RMSNorm (rmsnorm_row_kernel) for rows of nvec
// float4 (nvec <= 4096): nv float4 per lane and `threads` lanes per row.  Two
// float4 per lane where the row allows it, at most 16 waves; one per lane for
// few rows (decode), where more lanes per row win; with many rows of 129 to
// 256 float4 (hidden 1024) four per lane, one wave per row, which needs no
// LDS exchange and no barrier (measured at 2048 rows of 1024: 3.1 us against
// 3.5 for two waves of two).  The geometry fixes the order of the sum of
// squares, so every kernel that must reproduce the RMSNorm's bits takes it
// from here.
inline void rms_row_geometry(long rows, int nvec, int& nv, int& threads) {
    if (nvec <= 64 || (rows < 256 && nvec <= 1024)) nv = 1;
    else if (nvec > 128 && nvec <= 256) nv = 4;
    else nv = nvec <= 1024 * 2 ? 2 : 4;
    threads = ((nvec + nv - 1) / nv + 63) / 64 * 64;
}

// ---------------------------------------------- per-head q/k norm + RoPE
// Shared by the q/k norm kernels and the attention that applies them on the
// fly, so both produce the same bits.
// cos/sin of the rotation angles j0 .. j0+3 at position p: table row p when
// 0 <= p < tab_len (qwen3.cpp:463-469), else the fallback angle
// p * inv_freq[j] (qwen3.cpp:39-49).
__device__ __noinline__ float2 cos_sin_cold(float ang) { return make_float2(cosf(ang), sinf(ang)); }

__device__ __forceinline__ void rope_cs4(int p, int j0, const float* cos_tab, const float* sin_tab, int tab_len,
                                         const float* inv, float4& c, float4& s) {
    if (p >= 0 && p < tab_len) {
        c = *reinterpret_cast<const float4*>(cos_tab + (long)p * 64 + j0);
        s = *reinterpret_cast<const float4*>(sin_tab + (long)p * 64 + j0);
    } else {
        // one angle per trip through an out-of-line cosf/sinf: keeps the
        // code of the kernels that share this small (it is not the common path)
        const float pf = (float)p;
#pragma unroll 1
        for (int i = 0; i < 4; i++) {
            const float2 cs = cos_sin_cold(pf * inv[j0 + i]);
            const float cv = cs.x, sv = cs.y;
            c.x = i == 0 ? cv : c.x;
            c.y = i == 1 ? cv : c.y;
            c.z = i == 2 ? cv : c.z;
            c.w = i == 3 ? cv : c.w;
            s.x = i == 0 ? sv : s.x;
            s.y = i == 1 ? sv : s.y;
            s.z = i == 2 ? sv : s.z;
            s.w = i == 3 ? sv : s.w;
        }
    }
}

// One 128-wide head held by an aligned group of 16 lanes, lane l holding
// elements j0 = 4*(l%16) .. j0+3 in `l` and j0+64 .. j0+67 in `h`: the
// RMSNorm with gamma wl / wh (this lane's gammas; skipped when !has_w), then
// the half-split rotation; returns the rotated halves in ol / oh.  Every lane
// of the group calls it (the sum of squares is a group reduction).
__device__ __forceinline__ void norm_rope128_w(float4 l, float4 h, bool has_w, float4 wl, float4 wh, float4 c,
                                               float4 s, float eps, float4& ol, float4& oh) {
    float ss = 0.f;
    ss = fmaf(l.x, l.x, ss);
    ss = fmaf(l.y, l.y, ss);
    ss = fmaf(l.z, l.z, ss);
    ss = fmaf(l.w, l.w, ss);
    ss = fmaf(h.x, h.x, ss);
    ss = fmaf(h.y, h.y, ss);
    ss = fmaf(h.z, h.z, ss);
    ss = fmaf(h.w, h.w, ss);
    ss = group16_sum(ss);
    if (has_w) {
        const float sc = 1.0f / sqrtf(ss / 128.0f + eps);
        l.x = (l.x * sc) * wl.x;
        l.y = (l.y * sc) * wl.y;
        l.z = (l.z * sc) * wl.z;
        l.w = (l.w * sc) * wl.w;
        h.x = (h.x * sc) * wh.x;
        h.y = (h.y * sc) * wh.y;
        h.z = (h.z * sc) * wh.z;
        h.w = (h.w * sc) * wh.w;
    }
    ol.x = l.x * c.x - h.x * s.x;
    ol.y = l.y * c.y - h.y * s.y;
    ol.z = l.z * c.z - h.z * s.z;
    ol.w = l.w * c.w - h.w * s.w;
    oh.x = h.x * c.x + l.x * s.x;
    oh.y = h.y * c.y + l.y * s.y;
    oh.z = h.z * c.z + l.z * s.z;
    oh.w = h.w * c.w + l.w * s.w;
}

// The gammas of lane slice j0 of a 128-wide head (ones when w is null).
template <int DT>
__device__ __forceinline__ void head_gamma128(const void* w, int j0, float4& wl, float4& wh) {
    wl = wh = make_float4(1.f, 1.f, 1.f, 1.f);
    if (w) {
        wl = load_w4<DT>(w, j0);
        wh = load_w4<DT>(w, j0 + 64);
    }
}

// norm_rope128_w with the gammas read from w (element type DT; null skips
// the norm).
template <int DT>
__device__ __forceinline__ void norm_rope128(float4 l, float4 h, const void* w, float4 c, float4 s, int j0,
                                             float eps, float4& ol, float4& oh) {
    float4 wl, wh;
    head_gamma128<DT>(w, j0, wl, wh);
    norm_rope128_w(l, h, w != nullptr, wl, wh, c, s, eps, ol, oh);
}

}  // namespace anelm
