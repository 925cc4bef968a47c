// fp32 MFMA and raw-buffer helpers shared by the chunked gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace xm {

typedef float v4f __attribute__((ext_vector_type(4)));

// v_mfma_f32_16x16x4_f32: A[m][k] in lane m+16k, B[k][n] in lane n+16k,
// D[m][n] in lane n+16(m/4), register m%4.
__device__ __forceinline__ v4f Mfma(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f LdsF4(const float *p) { return *reinterpret_cast<const v4f *>(p); }
__device__ __forceinline__ void StF4(float *p, v4f v) { *reinterpret_cast<v4f *>(p) = v; }

// Raw buffer access: a wave-uniform descriptor (base address, size in bytes),
// per-lane byte offsets and an optional wave-uniform byte offset.  Loads
// whose per-lane plus scalar offset is at or beyond the size return zeros and
// stores there are dropped (the range check covers the sum: measured on
// gfx950, size 256 with scalar offset 128 drops per-lane offsets from 128 on),
// which masks tokens past the sequence end and columns past dv with no branch.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kRawBufferWord3 = 0x00020000;                       // untyped 32-bit data format
constexpr int kOutOfRange = static_cast<int>(0x80000000u);        // beyond any descriptor size used here
__device__ __forceinline__ Rsrc MakeRsrc(const float *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), static_cast<short>(0), bytes, kRawBufferWord3);
}
__device__ __forceinline__ v4f BufF4(Rsrc r, int voff, int soff) {
    return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float BufF(Rsrc r, int voff, int soff = 0) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void BufStF(Rsrc r, int voff, float x, int soff = 0) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, x), r, voff, soff, 0);
}
// Orders this wave's LDS accesses before and after (the LDS unit serves one
// wave's operations in order; this stops the compiler from moving them), so
// a wave can read back what its other lanes just wrote.
__device__ __forceinline__ void WaveSync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// A 64-bit value known to be equal in every lane, in SGPRs.
__device__ __forceinline__ size_t Uniform64(size_t x) {
    const unsigned lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(x));
    const unsigned hi = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(x >> 32));
    return (static_cast<size_t>(hi) << 32) | lo;
}
__device__ __forceinline__ float2 BufF2(Rsrc r, int voff, int soff = 0) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

}  // namespace xm
