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

// sum over aligned groups of 16 lanes
__device__ __forceinline__ float group16_sum(float v) {
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
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

}  // namespace anelm
