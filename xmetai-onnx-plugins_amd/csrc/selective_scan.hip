// SelectiveScanFn forward for gfx950 (CDNA4, wave64).
//
// Computes output 0 of the reference operator (selective_scan_fwd_kernel.cuh:
// 70-306): per channel (b,d) and state n,
//     delta' = softplus?(delta + bias),  h_t = exp2(delta'_t * A[d,n] * log2e) h_{t-1} + B_t delta'_t u_t,
//     y_t = D u_t + sum_n C_t h_t.
//
// Layout of the work (MI355X-first, not the reference's block scan):
//  * A lane owns SPL consecutive states of one channel and runs their
//    recurrences sequentially over the whole sequence, so every (t,n) costs
//    exactly one exp2 and four VALU ops; there is no cross-lane scan.
//  * LPC = ceil(N/SPL) lanes share a channel; a 256-thread workgroup owns
//    CPW = 256/LPC channels of one (batch, group), which share the B/C rows.
//  * The sequence is processed in tiles of kTile tokens.  Per tile the
//    workgroup loads u/delta rows and the B/C rows with coalesced 16-byte
//    loads (prefetched one tile ahead into registers), applies bias and
//    softplus once per (channel, token), and stages delta' and delta'*u in LDS.
//  * Each lane writes its partial sum over its states into LDS; the store
//    phase adds the LPC partials and D*u and writes y with 16-byte stores.
//  * z is never read: output 0 does not depend on it (reference
//    selective_scan_fwd_kernel.cuh:280 vs :296-299).
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "xm_hip.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 16;           // tokens per tile
constexpr int kRow = kTile + 4;     // LDS row stride in floats (padding breaks bank aliasing)
constexpr int kQ4 = kTile / 4;      // float4 groups per tile row

struct F4 {
    float v[4];
};

__device__ __forceinline__ F4 LoadRow4(const float *row, int t, int L, bool vec) {
    F4 r;
    if (vec && t + 3 < L) {
        float4 x = *reinterpret_cast<const float4 *>(row + t);
        r.v[0] = x.x; r.v[1] = x.y; r.v[2] = x.z; r.v[3] = x.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) r.v[e] = (t + e < L) ? row[t + e] : 0.0f;
    }
    return r;
}

__device__ __forceinline__ void StoreRow4(float *row, int t, int L, bool vec, const F4 &x) {
    if (vec && t + 3 < L) {
        *reinterpret_cast<float4 *>(row + t) = make_float4(x.v[0], x.v[1], x.v[2], x.v[3]);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (t + e < L) row[t + e] = x.v[e];
    }
}

__device__ __forceinline__ float Softplus(float x) {
    // reference selective_scan_fwd_kernel.cuh:157-159
    return x <= 20.0f ? log1pf(expf(x)) : x;
}

template <int LPC, int SPL, bool BVAR, bool CVAR>
__global__ __launch_bounds__(kThreads) void SelectiveScanFwdKernel(SelectiveScanParams p, int vec) {
    constexpr int CPW = kThreads / LPC;      // channels per workgroup
    constexpr int NP = LPC * SPL;            // padded state count
    constexpr int ITEMS = CPW * kQ4;         // (channel, 4-token) items per tile
    constexpr int IPT = (ITEMS + kThreads - 1) / kThreads;
    constexpr int NBC = (BVAR ? 1 : 0) + (CVAR ? 1 : 0);
    constexpr int BCPT = NBC == 0 ? 1 : (NBC * NP * kQ4 + kThreads - 1) / kThreads;

    __shared__ __attribute__((aligned(16))) float sDl[CPW * kRow];        // delta' per (channel, token)
    __shared__ __attribute__((aligned(16))) float sDu[CPW * kRow];        // delta' * u
    __shared__ __attribute__((aligned(16))) float sB[BVAR ? NP * kRow : 1];
    __shared__ __attribute__((aligned(16))) float sC[CVAR ? NP * kRow : 1];
    __shared__ __attribute__((aligned(16))) float sY[kThreads * kRow];    // per-lane partial outputs

    const int tid = threadIdx.x;
    const int L = p.seqlen;
    const int N = p.dstate;
    const int dpg = p.dim_per_group;
    const int ncb = (dpg + CPW - 1) / CPW;
    int wg = blockIdx.x;
    const int cb = wg % ncb;
    wg /= ncb;
    const int g = wg % p.groups_b;
    const int b = wg / p.groups_b;
    const int cbase = g * dpg + cb * CPW;    // first channel of this workgroup
    const int nvalid = min(CPW, dpg - cb * CPW);

    const size_t row0 = (static_cast<size_t>(b) * p.dim + cbase) * static_cast<size_t>(L);
    const float *__restrict__ ub = p.u + row0;
    const float *__restrict__ db = p.delta + row0;
    float *__restrict__ ob = p.out + row0;
    const float *__restrict__ Bb =
        BVAR ? p.B + (static_cast<size_t>(b) * p.groups_b + g) * static_cast<size_t>(N) * L : nullptr;
    const float *__restrict__ Cb =
        CVAR ? p.C + (static_cast<size_t>(b) * p.groups_c + (BVAR ? g : 0)) * static_cast<size_t>(N) * L : nullptr;
    const bool v4 = vec != 0;

    // ---- per-lane recurrence constants ------------------------------------
    const int lc = tid / LPC;   // channel of this lane within the workgroup
    const int lq = tid % LPC;   // which block of SPL states
    const bool lane_ok = lc < nvalid;
    const int dl = cbase + lc;
    float A2[SPL], h[SPL], bco[SPL], cco[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        const int n = lq * SPL + j;
        const bool ok = lane_ok && n < N;
        const size_t idx = static_cast<size_t>(dl) * N + n;
        A2[j] = ok ? p.A[idx] * kLog2eF : 0.0f;   // A_val *= kLog2e (kernel.cuh:170-178)
        bco[j] = (!BVAR && ok) ? p.B[idx] : 0.0f;
        cco[j] = (!CVAR && ok) ? p.C[idx] : 0.0f;
        if (!BVAR && !CVAR) bco[j] = bco[j] * cco[j];  // B*C folded (kernel.cuh:205-210)
        h[j] = 0.0f;
    }

    // Zero the padded state rows once; tiles only overwrite rows < N.
    if (BVAR)
        for (int i = tid; i < (NP - N) * kRow; i += kThreads) sB[N * kRow + i] = 0.0f;
    if (CVAR)
        for (int i = tid; i < (NP - N) * kRow; i += kThreads) sC[N * kRow + i] = 0.0f;

    // ---- tile loads (global -> registers) ----------------------------------
    F4 ureg[IPT], dreg[IPT], bcreg[BCPT];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int it = tid + k * kThreads;
            const int c = it / kQ4, t = t0 + (it % kQ4) * 4;
            if (it < ITEMS && c < nvalid) {
                ureg[k] = LoadRow4(ub + static_cast<size_t>(c) * L, t, L, v4);
                dreg[k] = LoadRow4(db + static_cast<size_t>(c) * L, t, L, v4);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) ureg[k].v[e] = dreg[k].v[e] = 0.0f;
            }
        }
        if (NBC > 0) {
            const int per = N * kQ4;
#pragma unroll
            for (int k = 0; k < BCPT; ++k) {
                const int it = tid + k * kThreads;
                if (it < NBC * per) {
                    const bool isB = BVAR && it < per;
                    const int r = it % per;
                    const float *base = isB ? Bb : Cb;
                    bcreg[k] = LoadRow4(base + static_cast<size_t>(r / kQ4) * L, t0 + (r % kQ4) * 4, L, v4);
                }
            }
        }
    };

    float bias[IPT], dsk[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = tid + k * kThreads;
        const int c = it / kQ4;
        const bool ok = it < ITEMS && c < nvalid;
        bias[k] = (ok && p.delta_bias) ? p.delta_bias[cbase + c] : 0.0f;
        dsk[k] = (ok && p.D) ? p.D[cbase + c] : 0.0f;
    }

    load_tile(0);
    for (int t0 = 0; t0 < L; t0 += kTile) {
        // ---- phase 1: bias, softplus, delta*u into LDS; keep D*u ------------
        F4 skip[IPT];
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int it = tid + k * kThreads;
            if (it < ITEMS) {
                const int c = it / kQ4, q4 = it % kQ4;
                F4 dlv, duv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = dreg[k].v[e] + bias[k];
                    if (p.delta_softplus) x = Softplus(x);
                    if (t0 + q4 * 4 + e >= L) x = 0.0f;   // past the end: a = 1, b = 0
                    dlv.v[e] = x;
                    duv.v[e] = x * ureg[k].v[e];
                    skip[k].v[e] = dsk[k] * ureg[k].v[e];
                }
                *reinterpret_cast<float4 *>(&sDl[c * kRow + q4 * 4]) = make_float4(dlv.v[0], dlv.v[1], dlv.v[2], dlv.v[3]);
                *reinterpret_cast<float4 *>(&sDu[c * kRow + q4 * 4]) = make_float4(duv.v[0], duv.v[1], duv.v[2], duv.v[3]);
            }
        }
        if (NBC > 0) {
            const int per = N * kQ4;
#pragma unroll
            for (int k = 0; k < BCPT; ++k) {
                const int it = tid + k * kThreads;
                if (it < NBC * per) {
                    const bool isB = BVAR && it < per;
                    const int r = it % per;
                    float *dst = (isB ? sB : sC) + (r / kQ4) * kRow + (r % kQ4) * 4;
                    *reinterpret_cast<float4 *>(dst) = make_float4(bcreg[k].v[0], bcreg[k].v[1], bcreg[k].v[2], bcreg[k].v[3]);
                }
            }
        }
        __syncthreads();

        // Prefetch the next tile while the recurrence runs.
        if (t0 + kTile < L) load_tile(t0 + kTile);

        // ---- phase 2: the recurrence over this tile --------------------------
        const float *rDl = sDl + lc * kRow;
        const float *rDu = sDu + lc * kRow;
        float *rY = sY + tid * kRow;
#pragma unroll
        for (int q4 = 0; q4 < kQ4; ++q4) {
            const float4 dl4 = *reinterpret_cast<const float4 *>(rDl + q4 * 4);
            const float4 du4 = *reinterpret_cast<const float4 *>(rDu + q4 * 4);
            const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
            const float duv[4] = {du4.x, du4.y, du4.z, du4.w};
            float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < SPL; ++j) {
                float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f}, cv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (BVAR) {
                    const float4 x = *reinterpret_cast<const float4 *>(sB + (lq * SPL + j) * kRow + q4 * 4);
                    bv[0] = x.x; bv[1] = x.y; bv[2] = x.z; bv[3] = x.w;
                }
                if (CVAR) {
                    const float4 x = *reinterpret_cast<const float4 *>(sC + (lq * SPL + j) * kRow + q4 * 4);
                    cv[0] = x.x; cv[1] = x.y; cv[2] = x.z; cv[3] = x.w;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = __builtin_amdgcn_exp2f(dlv[e] * A2[j]);
                    const float bt = BVAR ? bv[e] * duv[e] : duv[e];
                    h[j] = fmaf(a, h[j], bt);
                    float cc;
                    if (CVAR) cc = BVAR ? cv[e] : bco[j] * cv[e];
                    else cc = BVAR ? cco[j] : bco[j];
                    y[e] = fmaf(h[j], cc, y[e]);
                }
            }
            *reinterpret_cast<float4 *>(rY + q4 * 4) = make_float4(y[0], y[1], y[2], y[3]);
        }
        __syncthreads();

        // ---- phase 3: add the LPC partials and D*u, store y ------------------
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int it = tid + k * kThreads;
            if (it < ITEMS) {
                const int c = it / kQ4, q4 = it % kQ4;
                if (c < nvalid) {
                    F4 acc = skip[k];
#pragma unroll
                    for (int q = 0; q < LPC; ++q) {
                        const float4 x = *reinterpret_cast<const float4 *>(sY + (c * LPC + q) * kRow + q4 * 4);
                        acc.v[0] += x.x; acc.v[1] += x.y; acc.v[2] += x.z; acc.v[3] += x.w;
                    }
                    StoreRow4(ob + static_cast<size_t>(c) * L, t0 + q4 * 4, L, v4, acc);
                }
            }
        }
        // sY is rewritten only after the next phase-1 barrier; sDl/sDu/sB/sC
        // were last read before the barrier above, so no barrier is needed here.
    }
}

struct Config {
    int lpc, spl;
};

// States per lane and lanes per channel by dstate.  XM_SS_LPC overrides the
// lanes per channel for dstate <= 16 (1, 2, 4, 8 or 16), for tuning.
Config ChooseConfig(int N) {
    if (N <= 16) {
        const char *env = std::getenv("XM_SS_LPC");
        const int forced = env ? std::atoi(env) : 0;
        switch (forced) {
            case 8: return {8, 2};
            case 16: return {16, 1};
            case 2: if (N <= 8) return {2, 4}; break;
            case 1: if (N <= 4) return {1, 4}; break;
            default: break;
        }
        if (N <= 4) return {1, 4};
        if (N <= 8) return {2, 4};
        return {4, 4};
    }
    if (N <= 32) return {8, 4};
    if (N <= 64) return {16, 4};
    if (N <= 128) return {16, 8};
    return {16, 16};
}

template <int LPC, int SPL>
void LaunchLS(const SelectiveScanParams &p, int vec, dim3 grid, hipStream_t stream) {
    if (p.b_var && p.c_var)
        hipLaunchKernelGGL((SelectiveScanFwdKernel<LPC, SPL, true, true>), grid, dim3(kThreads), 0, stream, p, vec);
    else if (p.b_var)
        hipLaunchKernelGGL((SelectiveScanFwdKernel<LPC, SPL, true, false>), grid, dim3(kThreads), 0, stream, p, vec);
    else if (p.c_var)
        hipLaunchKernelGGL((SelectiveScanFwdKernel<LPC, SPL, false, true>), grid, dim3(kThreads), 0, stream, p, vec);
    else
        hipLaunchKernelGGL((SelectiveScanFwdKernel<LPC, SPL, false, false>), grid, dim3(kThreads), 0, stream, p, vec);
}

bool Aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

void LaunchSelectiveScan(const SelectiveScanParams &p, void *stream_v) {
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    const Config cfg = ChooseConfig(p.dstate);
    const int cpw = kThreads / cfg.lpc;
    const long long ncb = (p.dim_per_group + cpw - 1) / cpw;
    const long long blocks = ncb * p.groups_b * static_cast<long long>(p.batch);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "SelectiveScanFn launch exceeds the grid limit");
    const int vec = (p.seqlen % 4 == 0) && Aligned16(p.u) && Aligned16(p.delta) && Aligned16(p.out) &&
                    (!p.b_var || Aligned16(p.B)) && (!p.c_var || Aligned16(p.C));
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (cfg.lpc * 100 + cfg.spl) {
        case 104: LaunchLS<1, 4>(p, vec, grid, stream); break;
        case 204: LaunchLS<2, 4>(p, vec, grid, stream); break;
        case 404: LaunchLS<4, 4>(p, vec, grid, stream); break;
        case 802: LaunchLS<8, 2>(p, vec, grid, stream); break;
        case 1601: LaunchLS<16, 1>(p, vec, grid, stream); break;
        case 804: LaunchLS<8, 4>(p, vec, grid, stream); break;
        case 1604: LaunchLS<16, 4>(p, vec, grid, stream); break;
        case 1608: LaunchLS<16, 8>(p, vec, grid, stream); break;
        default: LaunchLS<16, 16>(p, vec, grid, stream); break;
    }
    XM_LAUNCH_CHECK("SelectiveScanFn");
}

}  // namespace xm
