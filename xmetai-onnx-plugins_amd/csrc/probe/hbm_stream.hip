// HBM streaming probe for gfx950: the "achievable bandwidth" denominator of
// the benchmark's roofline fractions.  Not part of the operator library; it is
// built as libxm_hbm_probe.so next to it.
//
// Two grid-stride kernels over 16-byte vectors: a copy (read + write) and a
// read-only sum.  Each thread keeps U independent 16-byte accesses in flight
// per iteration; a workgroup's U*256 vectors per iteration are contiguous, so
// every access instruction covers whole 128-byte lines.  NT selects the
// nontemporal (streaming) cache policy.  The benchmark sweeps grid size, U and
// NT and reports the best rate.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

template <int U, bool NT>
__global__ __launch_bounds__(256) void HbmCopyKernel(const v4f *__restrict__ src, v4f *__restrict__ dst, size_t n4) {
    const size_t step = static_cast<size_t>(gridDim.x) * U * 256;
    size_t i = static_cast<size_t>(blockIdx.x) * U * 256 + threadIdx.x;
    for (; i + (U - 1) * 256 < n4; i += step) {
        v4f v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * 256) : src[i + u * 256];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (NT) __builtin_nontemporal_store(v[u], dst + i + u * 256);
            else dst[i + u * 256] = v[u];
        }
    }
    for (int u = 0; u < U; ++u)   // the ragged end: whatever the loop left
        if (i + u * 256 < n4) dst[i + u * 256] = src[i + u * 256];
}

template <int U, bool NT>
__global__ __launch_bounds__(256) void HbmReadKernel(const v4f *__restrict__ src, size_t n4, float *sink) {
    const size_t step = static_cast<size_t>(gridDim.x) * U * 256;
    size_t i = static_cast<size_t>(blockIdx.x) * U * 256 + threadIdx.x;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (; i + (U - 1) * 256 < n4; i += step) {
        v4f v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * 256) : src[i + u * 256];
#pragma unroll
        for (int u = 0; u < U; ++u) acc += v[u];
    }
    for (int u = 0; u < U; ++u)
        if (i + u * 256 < n4) acc += src[i + u * 256];
    const float s = acc[0] + acc[1] + acc[2] + acc[3];
    if (s == 1234567.0f) sink[blockIdx.x] = s;   // keeps the loads; the value never occurs for the probe's data
}

template <int U, bool NT>
void LaunchCopy(const void *src, void *dst, size_t n4, int blocks, hipStream_t s) {
    hipLaunchKernelGGL((HbmCopyKernel<U, NT>), dim3(blocks), dim3(256), 0, s, static_cast<const v4f *>(src),
                       static_cast<v4f *>(dst), n4);
}

template <int U, bool NT>
void LaunchRead(const void *src, size_t n4, float *sink, int blocks, hipStream_t s) {
    hipLaunchKernelGGL((HbmReadKernel<U, NT>), dim3(blocks), dim3(256), 0, s, static_cast<const v4f *>(src), n4, sink);
}

bool Aligned(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

// Copies `bytes` (a multiple of 16, 16-byte aligned buffers) from src to dst
// on `stream` with `blocks` workgroups of 256 threads, `unroll` (1, 2, 4 or 8)
// vectors in flight per thread and nontemporal accesses when `nontemporal`.
// Returns 0, or -1 for arguments outside that set.
int xm_probe_hbm_copy(const void *src, void *dst, size_t bytes, int blocks, int unroll, int nontemporal,
                      void *stream) {
    if (bytes % 16 != 0 || !Aligned(src) || !Aligned(dst) || blocks <= 0) return -1;
    const size_t n4 = bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool nt = nontemporal != 0;
    switch (unroll) {
        case 1: nt ? LaunchCopy<1, true>(src, dst, n4, blocks, s) : LaunchCopy<1, false>(src, dst, n4, blocks, s); break;
        case 2: nt ? LaunchCopy<2, true>(src, dst, n4, blocks, s) : LaunchCopy<2, false>(src, dst, n4, blocks, s); break;
        case 4: nt ? LaunchCopy<4, true>(src, dst, n4, blocks, s) : LaunchCopy<4, false>(src, dst, n4, blocks, s); break;
        case 8: nt ? LaunchCopy<8, true>(src, dst, n4, blocks, s) : LaunchCopy<8, false>(src, dst, n4, blocks, s); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Reads `bytes` from src (same rules); `sink` is a device buffer of `blocks`
// floats that is written only if a workgroup's sum equals 1234567.
int xm_probe_hbm_read(const void *src, size_t bytes, float *sink, int blocks, int unroll, int nontemporal,
                      void *stream) {
    if (bytes % 16 != 0 || !Aligned(src) || blocks <= 0 || sink == nullptr) return -1;
    const size_t n4 = bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool nt = nontemporal != 0;
    switch (unroll) {
        case 1: nt ? LaunchRead<1, true>(src, n4, sink, blocks, s) : LaunchRead<1, false>(src, n4, sink, blocks, s); break;
        case 2: nt ? LaunchRead<2, true>(src, n4, sink, blocks, s) : LaunchRead<2, false>(src, n4, sink, blocks, s); break;
        case 4: nt ? LaunchRead<4, true>(src, n4, sink, blocks, s) : LaunchRead<4, false>(src, n4, sink, blocks, s); break;
        case 8: nt ? LaunchRead<8, true>(src, n4, sink, blocks, s) : LaunchRead<8, false>(src, n4, sink, blocks, s); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
