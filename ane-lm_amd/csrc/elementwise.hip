// Streaming elementwise ops for gfx950: residual add, SwiGLU, SiLU,
// mul-sigmoid, the bf16/fp16 weight converts and the embedding gather.
//
// Every op here is a pure stream (< 1 flop/byte).  The vector kernels move
// 16 bytes per lane per access and keep U independent 16-byte loads per
// stream in flight per lane before the first store, with a one-shot grid
// (one tile of 256*U vectors per workgroup, no grid-stride loop), so a
// launch has ~n/(256*U) workgroups -- far more than the 256 CUs.  U was
// chosen per kernel by measurement at the 8B prefill sizes (lighter
// workgroups won for SwiGLU and the convert).  Streamed inputs and
// write-once outputs use non-temporal loads and stores.
#include "anelm_common.hpp"

namespace anelm {

constexpr int kU_add = 1;   // residual add
constexpr int kU_silu = 1;  // SwiGLU
constexpr int kU_cvt = 1;   // bf16 -> fp16 (packed 16-bit arithmetic, see cvt_pair)

// ------------------------------------------------------------ residual add
// qwen3.cpp:516/:527: x = x + y, one IEEE add per element (bit-exact).
// x, y and the store all non-temporal: at 8192 rows of 4096 alone, 62.7 us
// against 65.0 with x read through the caches and 70.6 with everything
// cached; in the layer chain, where x was just written by the add + RMSNorm
// through the caches, it measured no slower (418.3 against 420.8 us per layer).
template <int kU>
__global__ __launch_bounds__(256) void residual_add_vec_kernel(float4* x, const float4* y, size_t n4) {
    const size_t base = (size_t)blockIdx.x * (256 * kU) + threadIdx.x;
    float4 a[kU], b[kU];
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n4) {
            a[i] = ld_nt(x + idx);
            b[i] = ld_nt(y + idx);
        }
    }
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n4) {
            float4 r;
            r.x = a[i].x + b[i].x;
            r.y = a[i].y + b[i].y;
            r.z = a[i].z + b[i].z;
            r.w = a[i].w + b[i].w;
            st_nt(x + idx, r);
        }
    }
}

__global__ __launch_bounds__(256) void residual_add_scalar_kernel(float* x, const float* y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        x[i] = x[i] + y[i];
}

// ------------------------------------------------------------ SiLU family
// silu_ref (anelm_common.hpp); SwiGLU multiplies by up
// (core/ane_runtime.cpp:393-395).

__device__ __forceinline__ float4 silu_mul4(float4 g, float4 u) {
    float4 r;
    r.x = silu_ref(g.x) * u.x;
    r.y = silu_ref(g.y) * u.y;
    r.z = silu_ref(g.z) * u.z;
    r.w = silu_ref(g.w) * u.w;
    return r;
}

template <int kU>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(float4* h, const float4* g, const float4* u, size_t n4) {
    const size_t base = (size_t)blockIdx.x * (256 * kU) + threadIdx.x;
    float4 a[kU], b[kU];
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n4) {
            a[i] = ld_nt(g + idx);
            b[i] = ld_nt(u + idx);
        }
    }
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n4) st_nt(h + idx, silu_mul4(a[i], b[i]));
    }
}

// strided rows (gate/up as slices of a wider buffer), any alignment
__global__ __launch_bounds__(256) void silu_mul_rows_kernel(float* h, const float* g, const float* u,
                                                            long rows, long inter, long ld_h, long ld_g,
                                                            long ld_u) {
    const long n = rows * inter;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const long r = i / inter, c = i % inter;
        h[r * ld_h + c] = silu_ref(g[r * ld_g + c]) * u[r * ld_u + c];
    }
}

// silu_vec_inplace (cpu_ops.cpp:7-14) and mul_sigmoid_inplace (:16-23):
// y = y / (1 + expf(-z)); silu is the case z = y.
__global__ __launch_bounds__(256) void mul_sigmoid_kernel(float* y, const float* z, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float t = expf(-z[i]) + 1.0f;
        y[i] = y[i] / t;
    }
}

// ------------------------------------------------------------ converts
// bf16 -> fp16 truncating (include/ane_lm/common.h:58-83), 8 elements per
// 16-byte vector, integer ops only.  The two halves of a 32-bit word are
// converted together with packed 16-bit instructions, from the magnitude
// a = b & 0x7FFF of each half (bf16 exponent field E = a >> 7, mantissa
// a & 0x7F; fp16 exponent field e = E - 112):
//   e >= 1 (a >= 0x3880): ((min(a, 0x4780) - 0x3800) << 3) -- the exponent
//     rebased and the 7 mantissa bits moved up 3; E >= 143 (e >= 31, with
//     infinities and NaNs) clamps to 0x7C00, the reference's +-inf;
//   e <= 0: ((mantissa | 0x80) << 3) >> (1 - e), the reference's truncating
//     subnormal shift ((m | 0x800000) >> (1 - e)) >> 13 on the fp32 mantissa
//     field m = mantissa << 16; shifts of 12 and more leave 0 (e < -10: the
//     reference's signed zero), so the shift is clamped to 15;
// then the sign bit.  bf16_to_f16_trunc is the same function one element at
// a time (scalar tails); both give the reference's value for all 65,536
// patterns.  Half the instructions of the per-element form: at one vector
// per lane the launch reaches the plain-copy rate.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pair(uint32_t w) {
    const u16x2 a = __builtin_bit_cast(u16x2, w) & (u16x2)(0x7FFF);
    const u16x2 nrm = (__builtin_elementwise_min(a, (u16x2)(0x4780)) - (u16x2)(0x3800)) << (u16x2)(3);
    const u16x2 sh = __builtin_elementwise_min((u16x2)(113) - (a >> (u16x2)(7)), (u16x2)(15));
    const u16x2 sub = (((a & (u16x2)(0x7F)) | (u16x2)(0x80)) << (u16x2)(3)) >> sh;
    // all ones in the halves with e >= 1 (a > 0x387F), zero elsewhere
    const u16x2 nz = __builtin_elementwise_min(__builtin_elementwise_sub_sat(a, (u16x2)(0x387F)), (u16x2)(1));
    const uint32_t mk = __builtin_bit_cast(uint32_t, (u16x2)(0) - nz);
    return (w & 0x80008000u) | (__builtin_bit_cast(uint32_t, nrm) & mk) | (__builtin_bit_cast(uint32_t, sub) & ~mk);
}

template <int kU>
__global__ __launch_bounds__(256) void bf16_to_f16_vec_kernel(uint4* dst, const uint4* src, size_t n8) {
    const size_t base = (size_t)blockIdx.x * (256 * kU) + threadIdx.x;
    uint4 a[kU];
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n8) a[i] = ld_nt(src + idx);
    }
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n8) {
            uint4 r;
            r.x = cvt_pair(a[i].x);
            r.y = cvt_pair(a[i].y);
            r.z = cvt_pair(a[i].z);
            r.w = cvt_pair(a[i].w);
            st_nt(dst + idx, r);
        }
    }
}

// Many tensors in one launch: the table of up to kCvtBatch tensors travels
// in the kernel arguments, so no device-side list is needed.  Each tensor is
// cut into tiles of 256 * 8 * kU elements; workgroup w finds its tensor by a
// binary search over the tile prefix (uniform, scalar) and converts its
// tile, the last tile of a tensor also taking the n % 8 tail element-wise.
// (A lookup in two rounds of independent scalar loads, every 8th entry then
// 8 neighbours, measured slower: 5.84 against 5.35 ms for the 8B set.)
constexpr int kCvtBatch = 128;
struct CvtTable {
    const uint16_t* src[kCvtBatch];
    uint16_t* dst[kCvtBatch];
    unsigned long long n[kCvtBatch];
    unsigned tile0[kCvtBatch + 1];  // first tile of each tensor; tile0[count] = tiles in the launch
    int count;
};

template <int kU>
__global__ __launch_bounds__(256) void bf16_to_f16_multi_kernel(const CvtTable t) {
    const unsigned tile = blockIdx.x;
    int lo = 0, hi = t.count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (t.tile0[mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    const size_t n = t.n[lo], n8 = n / 8;
    const uint4* src = reinterpret_cast<const uint4*>(t.src[lo]);
    uint4* dst = reinterpret_cast<uint4*>(t.dst[lo]);
    const size_t base = (size_t)(tile - t.tile0[lo]) * (256 * kU) + threadIdx.x;
    uint4 a[kU];
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n8) a[i] = ld_nt(src + idx);
    }
#pragma unroll
    for (int i = 0; i < kU; i++) {
        const size_t idx = base + (size_t)i * 256;
        if (idx < n8) {
            uint4 r;
            r.x = cvt_pair(a[i].x);
            r.y = cvt_pair(a[i].y);
            r.z = cvt_pair(a[i].z);
            r.w = cvt_pair(a[i].w);
            st_nt(dst + idx, r);
        }
    }
    const size_t tail = n8 * 8 + threadIdx.x;  // the last tile: elements n8*8 .. n-1
    if (tile + 1 == t.tile0[lo + 1] && tail < n) t.dst[lo][tail] = (uint16_t)bf16_to_f16_trunc(t.src[lo][tail]);
}

__global__ __launch_bounds__(256) void bf16_to_f16_scalar_kernel(uint16_t* dst, const uint16_t* src, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = (uint16_t)bf16_to_f16_trunc(src[i]);
}

template <bool F16>
__global__ __launch_bounds__(256) void widen_kernel(float* dst, const uint16_t* src, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = F16 ? f16_to_f32_exact(src[i]) : bf16_to_f32(src[i]);
}

// The same, 8 elements per thread (one 16-byte load, two 16-byte stores).
template <bool F16>
__global__ __launch_bounds__(256) void widen_vec_kernel(float4* dst, const uint4* src, size_t n8) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const uint4 u = ld_nt(src + i);
    auto w = [](uint32_t h) { return F16 ? f16_to_f32_exact(h) : bf16_to_f32(h); };
    st_nt(dst + 2 * i, make_float4(w(u.x & 0xFFFFu), w(u.x >> 16), w(u.y & 0xFFFFu), w(u.y >> 16)));
    st_nt(dst + 2 * i + 1, make_float4(w(u.z & 0xFFFFu), w(u.z >> 16), w(u.w & 0xFFFFu), w(u.w >> 16)));
}

// The Qwen3.5 (1+w) norm weight (core/safetensors.cpp:299-306): bf16 widened
// exactly, then + 1.0f in fp32, rounded to nearest even as the reference's
// `w[i] += 1.0f` is.  +-Inf stays +-Inf; a NaN comes out quieted with its
// sign and payload kept, which is what an IEEE add of a NaN operand returns
// on the CPUs the reference runs on, written out so it does not depend on
// the GPU's NaN propagation.
__global__ __launch_bounds__(256) void widen_plus1_kernel(float* dst, const uint16_t* src, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const uint32_t b = (uint32_t)src[i] << 16;
        const bool nan = (b & 0x7FFFFFFFu) > 0x7F800000u;
        dst[i] = nan ? __uint_as_float(b | 0x00400000u) : __uint_as_float(b) + 1.0f;
    }
}

// fp32 -> fp16 round to nearest even (the activation conversion at the ANE
// kernel inputs, core/ane_runtime.cpp:604-612, where arm64's __fp16 cast
// rounds to nearest even): the hardware conversion, whose mode is RNE.
__device__ __forceinline__ uint32_t f16_rne(float x) {
    const _Float16 h = (_Float16)x;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

__global__ __launch_bounds__(256) void narrow_vec_kernel(uint2* dst, const float4* src, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const float4 v = src[i];
        dst[i] = make_uint2(f16_rne(v.x) | (f16_rne(v.y) << 16), f16_rne(v.z) | (f16_rne(v.w) << 16));
    }
}

__global__ __launch_bounds__(256) void narrow_kernel(uint16_t* dst, const float* src, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = (uint16_t)f16_rne(src[i]);
}

// ------------------------------------------------------------ gather
// qwen3.cpp:498: x = E[id].  gridDim.y = ids; each block moves a slice of
// the row.  A bad id leaves its row unwritten and bumps *bad once.
template <int DT>
__global__ __launch_bounds__(256) void gather_vec_kernel(float* out, const void* table, const int32_t* ids,
                                                         long hidden, long vocab, int32_t* bad) {
    const long b = blockIdx.y;
    const int id = ids[b];
    if (id < 0 || id >= vocab) {
        if (bad && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(bad, 1);
        return;
    }
    float* o = out + b * hidden;
    if (DT == ANELM_F32) {
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(table) + (long)id * hidden);
        const long n4 = hidden / 4;
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256)
            reinterpret_cast<float4*>(o)[i] = src[i];
    } else {
        // 8 halves (16 bytes) in, 2 float4 out per lane
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(table) + (long)id * hidden);
        const long n8 = hidden / 8;
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n8; i += (long)gridDim.x * 256) {
            const uint4 v = src[i];
            float4 lo, hi;
            if (DT == ANELM_F16) {
                lo = make_float4(f16_to_f32_exact(v.x & 0xFFFFu), f16_to_f32_exact(v.x >> 16),
                                 f16_to_f32_exact(v.y & 0xFFFFu), f16_to_f32_exact(v.y >> 16));
                hi = make_float4(f16_to_f32_exact(v.z & 0xFFFFu), f16_to_f32_exact(v.z >> 16),
                                 f16_to_f32_exact(v.w & 0xFFFFu), f16_to_f32_exact(v.w >> 16));
            } else {
                lo = make_float4(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16),
                                 bf16_to_f32(v.y & 0xFFFFu), bf16_to_f32(v.y >> 16));
                hi = make_float4(bf16_to_f32(v.z & 0xFFFFu), bf16_to_f32(v.z >> 16),
                                 bf16_to_f32(v.w & 0xFFFFu), bf16_to_f32(v.w >> 16));
            }
            reinterpret_cast<float4*>(o)[2 * i] = lo;
            reinterpret_cast<float4*>(o)[2 * i + 1] = hi;
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void gather_scalar_kernel(float* out, const void* table, const int32_t* ids,
                                                            long hidden, long vocab, int32_t* bad) {
    const long b = blockIdx.y;
    const int id = ids[b];
    if (id < 0 || id >= vocab) {
        if (bad && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(bad, 1);
        return;
    }
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < hidden; i += (long)gridDim.x * 256)
        out[b * hidden + i] = load_w<DT>(table, (long)id * hidden + i);
}

static unsigned grid_for(size_t work_items, size_t per_block) {
    size_t g = (work_items + per_block - 1) / per_block;
    return (unsigned)(g == 0 ? 1 : g);
}

static unsigned grid_stride_blocks(size_t n) {
    size_t g = (n + 255) / 256;
    if (g > 16384) g = 16384;
    return (unsigned)(g == 0 ? 1 : g);
}

}  // namespace anelm

using namespace anelm;

extern "C" int anelm_residual_add(float* x, const float* y, size_t n, void* stream) {
    if (!x || !y) return fail(ANELM_ERR_INVALID, "anelm_residual_add: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_residual_add: n == 0");
    clear_error();
    hipStream_t st = as_stream(stream);
    if (n % 4 == 0 && aligned16(x) && aligned16(y)) {
        const size_t n4 = n / 4;
        residual_add_vec_kernel<kU_add><<<grid_for(n4, 256 * kU_add), 256, 0, st>>>(reinterpret_cast<float4*>(x),
                                                                         reinterpret_cast<const float4*>(y), n4);
    } else {
        residual_add_scalar_kernel<<<grid_stride_blocks(n), 256, 0, st>>>(x, y, n);
    }
    return launch_status("residual_add");
}

extern "C" int anelm_silu_mul(float* h, const float* g, const float* u, long rows, long inter, long ld_h,
                              long ld_g, long ld_u, void* stream) {
    if (!h || !g || !u) return fail(ANELM_ERR_INVALID, "anelm_silu_mul: null pointer");
    if (rows <= 0 || inter <= 0) return fail(ANELM_ERR_INVALID, "anelm_silu_mul: rows=%ld inter=%ld", rows, inter);
    if (ld_h < inter || ld_g < inter || ld_u < inter) return fail(ANELM_ERR_INVALID, "anelm_silu_mul: ld < inter");
    clear_error();
    hipStream_t st = as_stream(stream);
    const size_t n = (size_t)rows * (size_t)inter;
    const bool contiguous = (ld_h == inter && ld_g == inter && ld_u == inter) || rows == 1;
    if (contiguous && n % 4 == 0 && aligned16(h) && aligned16(g) && aligned16(u)) {
        const size_t n4 = n / 4;
        silu_mul_vec_kernel<kU_silu><<<grid_for(n4, 256 * kU_silu), 256, 0, st>>>(
            reinterpret_cast<float4*>(h), reinterpret_cast<const float4*>(g), reinterpret_cast<const float4*>(u), n4);
    } else {
        silu_mul_rows_kernel<<<grid_stride_blocks(n), 256, 0, st>>>(h, g, u, rows, inter, ld_h, ld_g, ld_u);
    }
    return launch_status("silu_mul");
}

extern "C" int anelm_silu(float* x, size_t n, void* stream) {
    if (!x) return fail(ANELM_ERR_INVALID, "anelm_silu: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_silu: n == 0");
    clear_error();
    mul_sigmoid_kernel<<<grid_stride_blocks(n), 256, 0, as_stream(stream)>>>(x, x, n);
    return launch_status("silu");
}

extern "C" int anelm_mul_sigmoid(float* y, const float* z, size_t n, void* stream) {
    if (!y || !z) return fail(ANELM_ERR_INVALID, "anelm_mul_sigmoid: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_mul_sigmoid: n == 0");
    clear_error();
    mul_sigmoid_kernel<<<grid_stride_blocks(n), 256, 0, as_stream(stream)>>>(y, z, n);
    return launch_status("mul_sigmoid");
}

extern "C" int anelm_bf16_to_f16(uint16_t* dst, const uint16_t* src, size_t n, void* stream) {
    if (!dst || !src) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f16: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f16: n == 0");
    clear_error();
    hipStream_t st = as_stream(stream);
    if (n % 8 == 0 && aligned16(dst) && aligned16(src)) {
        const size_t n8 = n / 8;
        bf16_to_f16_vec_kernel<kU_cvt><<<grid_for(n8, 256 * kU_cvt), 256, 0, st>>>(reinterpret_cast<uint4*>(dst),
                                                                        reinterpret_cast<const uint4*>(src), n8);
    } else {
        bf16_to_f16_scalar_kernel<<<grid_stride_blocks(n), 256, 0, st>>>(dst, src, n);
    }
    return launch_status("bf16_to_f16");
}

template <bool F16>
static void launch_widen(float* dst, const uint16_t* src, size_t n, hipStream_t st) {
    if (n % 8 == 0 && aligned16(dst) && aligned16(src))
        widen_vec_kernel<F16><<<grid_for(n / 8, 256), 256, 0, st>>>(reinterpret_cast<float4*>(dst),
                                                                    reinterpret_cast<const uint4*>(src), n / 8);
    else
        widen_kernel<F16><<<grid_stride_blocks(n), 256, 0, st>>>(dst, src, n);
}

extern "C" int anelm_bf16_to_f16_multi(uint16_t* const* dst, const uint16_t* const* src, const size_t* n, int count,
                                       void* stream) {
    if (count < 0 || (count > 0 && (!dst || !src || !n))) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f16_multi: arguments");
    for (int i = 0; i < count; i++)
        if (n[i] > 0 && (!dst[i] || !src[i])) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f16_multi: null tensor %d", i);
    clear_error();
    hipStream_t st = as_stream(stream);
    constexpr size_t kTile = 256 * 8 * kU_cvt;
    CvtTable t;
    t.count = 0;
    t.tile0[0] = 0;
    auto flush = [&]() -> int {
        if (t.count == 0) return ANELM_OK;
        bf16_to_f16_multi_kernel<kU_cvt><<<dim3(t.tile0[t.count]), dim3(256), 0, st>>>(t);
        t.count = 0;
        return launch_status("bf16_to_f16_multi");
    };
    for (int i = 0; i < count; i++) {
        if (n[i] == 0) continue;
        if (!aligned16(dst[i]) || !aligned16(src[i])) {  // rare: its own launch, element-wise
            int rc = flush();
            if (rc) return rc;
            if ((rc = anelm_bf16_to_f16(dst[i], src[i], n[i], stream))) return rc;
            continue;
        }
        const size_t tiles = (n[i] + kTile - 1) / kTile;
        if (tiles > 0x7FFFFFFFu) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f16_multi: tensor %d too large", i);
        if (t.count == kCvtBatch || (size_t)t.tile0[t.count] + tiles > 0x7FFFFFFFu) {
            const int rc = flush();
            if (rc) return rc;
        }
        t.src[t.count] = src[i];
        t.dst[t.count] = dst[i];
        t.n[t.count] = n[i];
        t.tile0[t.count + 1] = t.tile0[t.count] + (unsigned)tiles;
        t.count++;
    }
    return flush();
}

extern "C" int anelm_bf16_to_f32(float* dst, const uint16_t* src, size_t n, void* stream) {
    if (!dst || !src) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f32: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f32: n == 0");
    clear_error();
    launch_widen<false>(dst, src, n, as_stream(stream));
    return launch_status("bf16_to_f32");
}

extern "C" int anelm_bf16_to_f32_plus1(float* dst, const uint16_t* src, size_t n, void* stream) {
    if (!dst || !src) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f32_plus1: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_bf16_to_f32_plus1: n == 0");
    clear_error();
    widen_plus1_kernel<<<grid_stride_blocks(n), 256, 0, as_stream(stream)>>>(dst, src, n);
    return launch_status("bf16_to_f32_plus1");
}

extern "C" int anelm_f32_to_f16(uint16_t* dst, const float* src, size_t n, void* stream) {
    if (!dst || !src) return fail(ANELM_ERR_INVALID, "anelm_f32_to_f16: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_f32_to_f16: n == 0");
    clear_error();
    if (n % 4 == 0 && aligned16(src) && aligned8(dst))
        narrow_vec_kernel<<<grid_stride_blocks(n / 4), 256, 0, as_stream(stream)>>>(
            reinterpret_cast<uint2*>(dst), reinterpret_cast<const float4*>(src), n / 4);
    else
        narrow_kernel<<<grid_stride_blocks(n), 256, 0, as_stream(stream)>>>(dst, src, n);
    return launch_status("f32_to_f16");
}

extern "C" int anelm_f16_to_f32(float* dst, const uint16_t* src, size_t n, void* stream) {
    if (!dst || !src) return fail(ANELM_ERR_INVALID, "anelm_f16_to_f32: null pointer");
    if (n == 0) return fail(ANELM_ERR_INVALID, "anelm_f16_to_f32: n == 0");
    clear_error();
    launch_widen<true>(dst, src, n, as_stream(stream));
    return launch_status("f16_to_f32");
}

template <int DT>
static void launch_gather(float* out, const void* table, const int32_t* ids, long n_ids, long hidden,
                          long vocab, int32_t* bad, hipStream_t st) {
    const int esz = DT == ANELM_F32 ? 4 : 2;
    const long per_vec = DT == ANELM_F32 ? 4 : 8;
    const bool vec = hidden % per_vec == 0 && aligned16(out) && aligned16(table) &&
                     ((hidden * esz) % 16 == 0);
    const long units = vec ? hidden / per_vec : hidden;
    long bx = (units + 255) / 256;
    if (bx > 64) bx = 64;
    const dim3 grd((unsigned)bx, (unsigned)n_ids);
    if (vec) gather_vec_kernel<DT><<<grd, 256, 0, st>>>(out, table, ids, hidden, vocab, bad);
    else gather_scalar_kernel<DT><<<grd, 256, 0, st>>>(out, table, ids, hidden, vocab, bad);
}

extern "C" int anelm_embed_gather(float* out, const void* table, int table_dtype, const int32_t* ids, long n_ids,
                                  long hidden, long vocab, int32_t* bad_count, void* stream) {
    if (!out || !table || !ids) return fail(ANELM_ERR_INVALID, "anelm_embed_gather: null pointer");
    if (n_ids <= 0 || hidden <= 0 || vocab <= 0) return fail(ANELM_ERR_INVALID, "anelm_embed_gather: empty");
    if (n_ids > 65535) return fail(ANELM_ERR_INVALID, "anelm_embed_gather: n_ids %ld > 65535", n_ids);
    clear_error();
    hipStream_t st = as_stream(stream);
    switch (table_dtype) {
        case ANELM_F32: launch_gather<ANELM_F32>(out, table, ids, n_ids, hidden, vocab, bad_count, st); break;
        case ANELM_F16: launch_gather<ANELM_F16>(out, table, ids, n_ids, hidden, vocab, bad_count, st); break;
        case ANELM_BF16: launch_gather<ANELM_BF16>(out, table, ids, n_ids, hidden, vocab, bad_count, st); break;
        default: return fail(ANELM_ERR_INVALID, "anelm_embed_gather: unknown dtype %d", table_dtype);
    }
    return launch_status("embed_gather");
}
