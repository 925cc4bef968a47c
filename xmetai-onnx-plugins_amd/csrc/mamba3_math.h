// Scalar math shared by the Mamba3SisoFn kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include "xm_hip.h"

namespace xm {
namespace m3 {

constexpr float kPiF = 3.14159265358979323846f;                     // reference kPi (mamba3_siso_fwd.cu:15)
constexpr double kTwoPiF = 2.0 * static_cast<double>(kPiF);         // reference kTwoPi = 2 * kPi: the wrap period
constexpr double kRevPerRad = 0.15915494309189533577;               // 1 / (2 pi): radians -> revolutions
constexpr double kInvTwoPiF = 1.0 / kTwoPiF;
constexpr double kRevPerTurn = kTwoPiF * kRevPerRad;                 // turns of the wrap period -> revolutions of 2 pi

// 1 / (1 + e^-x) with the hardware exp and reciprocal (about 2 ulp).
__device__ __forceinline__ float FastSigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// tanh without branches: the odd Taylor series to x^9 below |x| = 0.25
// (truncation < 1e-8 relative), above it 1 - 2 / (e^{2|x|} + 1) with the
// hardware exp2 and reciprocal (about 5e-7 relative near 0.25, less above).
__device__ __forceinline__ float TanhF(float x) {
    const float ax = fabsf(x), x2 = ax * ax;
    float p = fmaf(x2, 62.0f / 2835.0f, -17.0f / 315.0f);
    p = fmaf(x2, p, 2.0f / 15.0f);
    p = fmaf(x2, p, -1.0f / 3.0f);
    const float small = fmaf(ax, x2 * p, ax);
    const float e = __builtin_amdgcn_exp2f(fminf(ax * (2.0f * kLog2eF), 126.0f));
    const float big = fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
    return copysignf(ax < 0.25f ? small : big, x);
}

}  // namespace m3
}  // namespace xm
