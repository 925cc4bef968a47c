// HIP error mapping and small device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "xm_common.h"

#define XM_HIP_CHECK(expr)                                                                         \
    do {                                                                                           \
        hipError_t xm_err_ = (expr);                                                               \
        if (xm_err_ != hipSuccess)                                                                 \
            throw ::xm::Error(XM_ERR_DEVICE, std::string(#expr) + " failed: " + hipGetErrorString(xm_err_)); \
    } while (0)

// Reports a failed launch (reference: XM_CUDA_KERNEL_CHECK, cuda_common.h:27-36).
namespace xm {
// The HIP error this call's launches left on the thread, consumed; hipSuccess
// when there is none, or when the pending error is the one the caller had
// left before the call (ResetLaunches notes it): that one stays for the
// caller's own check.
hipError_t TakeLaunchError();
}  // namespace xm

#define XM_LAUNCH_CHECK(what)                                                                      \
    do {                                                                                           \
        hipError_t xm_err_ = ::xm::TakeLaunchError();                                              \
        if (xm_err_ != hipSuccess)                                                                 \
            throw ::xm::Error(XM_ERR_DEVICE, std::string(what) + " kernel launch failed: " + hipGetErrorString(xm_err_)); \
    } while (0)

namespace xm {

// Raises `kernel`'s dynamic-LDS limit to `bytes` on the current device the
// first time a launch needs it; later launches skip the runtime call.
void EnsureDynamicLds(const void *kernel, int bytes);

constexpr float kLog2eF = 1.4426950408889634f;  // M_LOG2E as float

// Moves `x` across lanes with a DPP control (row-local patterns only).
template <int CTRL>
__device__ __forceinline__ float DppF(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true));
}

// Sum over the 16 lanes of a DPP row, result in every lane of the row.
// xor 1 and xor 2 (quad_perm), xor 7 (row_half_mirror), xor 8 (row_ror:8)
// span all 16 lanes; each step folds into one v_add_f32_dpp.
__device__ __forceinline__ float RowSum16(float x) {
    x += DppF<0xB1>(x);   // quad_perm [1,0,3,2]
    x += DppF<0x4E>(x);   // quad_perm [2,3,0,1]
    x += DppF<0x141>(x);  // row_half_mirror
    x += DppF<0x128>(x);  // row_ror:8
    return x;
}

// Sum over 64 lanes, result in every lane.  After the row sum every lane of
// row r holds that row's sum; the GFX9 broadcast DPP controls then add row 0
// into row 1 and row 2 into row 3 (row_bcast:15, rows 1 and 3 enabled), and
// lane 31 (rows 0+1) into rows 2 and 3 (row_bcast:31), so lane 63 holds the
// total, which readlane returns to every lane.  No LDS traffic.
__device__ __forceinline__ float WaveSum64(float x) {
    x = RowSum16(x);
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xa, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xc, 0xf, false));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

__device__ __forceinline__ double WaveSum64d(double x) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) x += __shfl_xor(x, o);
    return x;
}

// KT consecutive floats of LDS into registers, 16 or 8 bytes at a time.
template <int KT>
__device__ __forceinline__ void LoadKeys(const float *src, float (&x)[KT]) {
    if constexpr (KT % 4 == 0) {
#pragma unroll
        for (int j = 0; j < KT; j += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(src + j);
            x[j] = v.x; x[j + 1] = v.y; x[j + 2] = v.z; x[j + 3] = v.w;
        }
    } else if constexpr (KT % 2 == 0) {
#pragma unroll
        for (int j = 0; j < KT; j += 2) {
            const float2 v = *reinterpret_cast<const float2 *>(src + j);
            x[j] = v.x; x[j + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int j = 0; j < KT; ++j) x[j] = src[j];
    }
}

// MI355X deals the workgroups of a launch round-robin to its 8 XCDs
// (workgroup x runs on XCD x % 8), and each XCD has its own L2.  This maps
// the hardware index to a logical one under which XCD j owns one contiguous
// range of logical indices, so workgroups that read the same data (adjacent
// logical indices) share an L2 instead of fetching it once per XCD.  It is a
// bijection on [0, n) for any n.
constexpr int kNumXcds = 8;
__device__ __forceinline__ int XcdLocalBlock(int x, int n) {
    const int per = n / kNumXcds, rem = n % kNumXcds;
    const int xcd = x % kNumXcds, slot = x / kNumXcds;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

}  // namespace xm
