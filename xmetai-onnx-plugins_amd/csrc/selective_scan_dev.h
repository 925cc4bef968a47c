// Device helpers shared by the SelectiveScanFn kernels (single-pass and
// sequence-parallel): 16-bit storage conversions, four-token row loads and
// stores, softplus, and the lane-swap reductions over the state lanes of a
// channel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "xm_hip.h"

namespace xm {
namespace ssdev {

// Sums of four values (tokens 0..3) over the 8 lanes {c, c+8, ..., c+56} of
// one channel c = lane % 8, with the gfx950 lane-swap instructions:
// permlane32_swap(a, b) yields [a.lo32, b.lo32] and [a.hi32, b.hi32], and
// permlane16_swap(a, b) yields [a.r0, b.r0, a.r2, b.r2] and [a.r1, b.r1, a.r3,
// b.r3] (r = 16-lane row), so adding the two halves of each swap halves the
// number of lanes and of values at once.  Seven instructions instead of the
// twelve of four separate 3-step reductions.  On return every lane of row r
// holds the channel sum of token {0, 2, 1, 3}[r] (see SwapReducedToken).
__device__ __forceinline__ float SwapReduce8x4(const float (&y)[4]) {
    const auto p01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(y[0]), __float_as_uint(y[1]), false, false);
    const auto p23 = __builtin_amdgcn_permlane32_swap(__float_as_uint(y[2]), __float_as_uint(y[3]), false, false);
    const float y01 = __uint_as_float(p01[0]) + __uint_as_float(p01[1]);   // lanes 0-31: y0, 32-63: y1
    const float y23 = __uint_as_float(p23[0]) + __uint_as_float(p23[1]);   // lanes 0-31: y2, 32-63: y3
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(y01), __float_as_uint(y23), false, false);
    const float z = __uint_as_float(q[0]) + __uint_as_float(q[1]);         // rows: y0, y2, y1, y3
    return z + DppF<0x128>(z);                                             // lanes c and c+8 of a row
}

// The same for 4 lanes per channel, {c, c+16, c+32, c+48} with c = lane % 16:
// the two swap stages alone reduce over the 4 lanes (six instructions).
__device__ __forceinline__ float SwapReduce4x4(const float (&y)[4]) {
    const auto p01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(y[0]), __float_as_uint(y[1]), false, false);
    const auto p23 = __builtin_amdgcn_permlane32_swap(__float_as_uint(y[2]), __float_as_uint(y[3]), false, false);
    const float y01 = __uint_as_float(p01[0]) + __uint_as_float(p01[1]);
    const float y23 = __uint_as_float(p23[0]) + __uint_as_float(p23[1]);
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(y01), __float_as_uint(y23), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__device__ __forceinline__ int SwapReducedToken(int lane) {
    const int r = lane >> 4;
    return ((r & 1) << 1) | (r >> 1);
}

struct F4 {
    float v[4];
};

// bfloat16 storage: the upper 16 bits of an fp32.
struct Bf16 {
    uint16_t bits;
};
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float ToF(float x) { return x; }
__device__ __forceinline__ float ToF(_Float16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float ToF(Bf16 x) { return __uint_as_float(static_cast<uint32_t>(x.bits) << 16); }

template <typename IT>
__device__ __forceinline__ IT FromF(float x);
template <>
__device__ __forceinline__ float FromF<float>(float x) { return x; }
template <>
__device__ __forceinline__ _Float16 FromF<_Float16>(float x) { return static_cast<_Float16>(x); }   // nearest even
template <>
__device__ __forceinline__ Bf16 FromF<Bf16>(float x) {   // nearest even; a NaN stays a (quiet) NaN
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return Bf16{static_cast<uint16_t>((u >> 16) | 0x40u)};
    return Bf16{static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16)};
}

// Four consecutive tokens t..t+3 of a row.  The guarded form clamps every
// address into the row and zeroes the lanes past the end with selects, so it
// has no branches (branches around loads make the compiler wait on each one,
// which would serialise the one-tile-ahead prefetch).
// (16 bytes of fp32 or 8 bytes of 16-bit data per vector access)
template <typename IT>
__device__ __forceinline__ F4 LoadRow4Fast(const IT *row, int t) {
    if constexpr (sizeof(IT) == 4) {
        const float4 x = *reinterpret_cast<const float4 *>(row + t);
        return F4{{x.x, x.y, x.z, x.w}};
    } else if constexpr (std::is_same_v<IT, _Float16>) {
        const h4 x = *reinterpret_cast<const h4 *>(row + t);
        return F4{{static_cast<float>(x[0]), static_cast<float>(x[1]), static_cast<float>(x[2]),
                   static_cast<float>(x[3])}};
    } else {
        const uint2 x = *reinterpret_cast<const uint2 *>(row + t);
        return F4{{__uint_as_float(x.x << 16), __uint_as_float(x.x & 0xffff0000u), __uint_as_float(x.y << 16),
                   __uint_as_float(x.y & 0xffff0000u)}};
    }
}

template <typename IT>
__device__ __forceinline__ F4 LoadRow4Guarded(const IT *row, int t, int L, bool ok) {
    F4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float v = ToF(row[min(t + e, L - 1)]);
        r.v[e] = (ok && t + e < L) ? v : 0.0f;
    }
    return r;
}

// Four elements at byte offset voff + soff of a raw buffer (a wave-uniform
// descriptor, a per-lane offset and a wave-uniform one), converted to fp32 /
// from fp32 (nearest even).  The offsets are in range by construction.
typedef __amdgpu_buffer_rsrc_t SsRsrc;
// A per-lane offset beyond any descriptor size used here: a store there is
// dropped (the bounds check of a raw buffer).
constexpr int kSsDropOffset = static_cast<int>(0x80000000u);
typedef unsigned SsU2 __attribute__((ext_vector_type(2)));
typedef unsigned SsU4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ SsRsrc SsRowsRsrc(const void *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), bytes, 0x00020000);
}
template <typename IT>
__device__ __forceinline__ F4 SsBufLoad4(SsRsrc r, int voff, int soff) {
    if constexpr (sizeof(IT) == 4) {
        const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
        return F4{{__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z), __uint_as_float(x.w)}};
    } else if constexpr (std::is_same_v<IT, _Float16>) {
        const h4 x = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
        return F4{{static_cast<float>(x[0]), static_cast<float>(x[1]), static_cast<float>(x[2]),
                   static_cast<float>(x[3])}};
    } else {
        const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
        return F4{{__uint_as_float(x.x << 16), __uint_as_float(x.x & 0xffff0000u), __uint_as_float(x.y << 16),
                   __uint_as_float(x.y & 0xffff0000u)}};
    }
}
template <typename IT>
__device__ __forceinline__ void SsBufStore4(SsRsrc r, int voff, int soff, const F4 &x) {
    if constexpr (sizeof(IT) == 4) {
        const SsU4 y{__float_as_uint(x.v[0]), __float_as_uint(x.v[1]), __float_as_uint(x.v[2]), __float_as_uint(x.v[3])};
        __builtin_amdgcn_raw_buffer_store_b128(y, r, voff, soff, 0);
    } else if constexpr (std::is_same_v<IT, _Float16>) {
        h4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = FromF<_Float16>(x.v[e]);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(SsU2, y), r, voff, soff, 0);
    } else {
        const unsigned lo = static_cast<uint32_t>(FromF<Bf16>(x.v[0]).bits) | (static_cast<uint32_t>(FromF<Bf16>(x.v[1]).bits) << 16);
        const unsigned hi = static_cast<uint32_t>(FromF<Bf16>(x.v[2]).bits) | (static_cast<uint32_t>(FromF<Bf16>(x.v[3]).bits) << 16);
        __builtin_amdgcn_raw_buffer_store_b64(SsU2{lo, hi}, r, voff, soff, 0);
    }
}

template <typename IT>
__device__ __forceinline__ void StoreRow4Fast(IT *row, int t, const F4 &x) {
    if constexpr (sizeof(IT) == 4) {
        *reinterpret_cast<float4 *>(row + t) = make_float4(x.v[0], x.v[1], x.v[2], x.v[3]);
    } else if constexpr (std::is_same_v<IT, _Float16>) {
        h4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = FromF<_Float16>(x.v[e]);
        *reinterpret_cast<h4 *>(row + t) = y;
    } else {
        uint2 y;
        y.x = static_cast<uint32_t>(FromF<Bf16>(x.v[0]).bits) | (static_cast<uint32_t>(FromF<Bf16>(x.v[1]).bits) << 16);
        y.y = static_cast<uint32_t>(FromF<Bf16>(x.v[2]).bits) | (static_cast<uint32_t>(FromF<Bf16>(x.v[3]).bits) << 16);
        *reinterpret_cast<uint2 *>(row + t) = y;
    }
}

template <typename IT>
__device__ __forceinline__ void StoreRow4(IT *row, int t, int L, bool vec, const F4 &x) {
    if (vec && t + 3 < L) {
        StoreRow4Fast(row, t, x);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (t + e < L) row[t + e] = FromF<IT>(x.v[e]);
    }
}

// softplus of the reference (selective_scan_fwd_kernel.cuh:157-159):
// x <= 20 ? log1p(exp(x)) : x, evaluated as max(x, 0) + log1p(t) with
// t = exp(-|x|) <= 1 on the hardware exp2/log2 (v_exp_f32, v_log_f32).
// u = 1 + t rounds with error c = (u - 1) - t, exact by Fast2Sum (Dekker,
// 1971) since t <= 1; log1p(t) = log(u) + log(1 - c/u) ~= log(u) - c, where
// dropping 1/u in [1/2, 1] changes the result by |c| t/u, under 2^-24
// relative.  For x > 20 the log term is below exp(-20) < ulp(x)/2, so the sum
// rounds to x exactly, the reference's other branch; +-inf and NaN pass
// through as in the reference.  Twelve issue slots against seventeen for
// log(1+e) * e / ((1+e) - 1) with its branches.
__device__ __forceinline__ float Softplus(float x) {
    constexpr float kLn2 = 0.69314718055994531f;
    const float t = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2eF);
    const float u = 1.0f + t;
    const float c = (u - 1.0f) - t;
    return fmaxf(x, 0.0f) + fmaf(__builtin_amdgcn_logf(u), kLn2, -c);
}


template <typename IT>
constexpr const char *TypeTag() {
    return sizeof(IT) == 4 ? "float" : (std::is_same_v<IT, _Float16> ? "half" : "bfloat16");
}

}  // namespace ssdev
}  // namespace xm
