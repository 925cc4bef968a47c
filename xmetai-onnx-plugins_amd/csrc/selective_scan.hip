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
//  * The sequence is processed in tiles of 32 tokens.  Per tile the
//    workgroup loads u/delta rows and the B/C rows with coalesced 16-byte
//    loads (prefetched one tile ahead into registers), applies bias and
//    softplus once per (channel, token), and stages delta' and delta'*u in LDS.
//  * The LPC partial sums over states are added across lanes with DPP; one
//    lane per channel writes them to LDS and the store phase adds D*u and
//    writes y with 16-byte stores.
//  * z is never read: output 0 does not depend on it (reference
//    selective_scan_fwd_kernel.cuh:280 vs :296-299).
//  * The data tensors (u, delta, variable B/C, y) are fp32, or float16 /
//    bfloat16 as in the reference's half and bfloat16 instantiations
//    (input_t; A, D, bias, constant B/C are weight_t = fp32): loads convert
//    to fp32, the arithmetic is fp32, y is rounded to nearest even.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "xm_hip.h"
#include "xm_params.h"
#include "selective_scan_dev.h"

namespace xm {
namespace {

using namespace ssdev;

constexpr int kThreads = 256;
// Sequence-split selection: single-pass workgroups below this count (one per
// CU), sequences at least this long.
constexpr long long kSegMaxChannelBlocks = 256;
constexpr int kSegMinSeqlen = 256;

// Tokens per tile: 32 fp32 = one 128-byte line per (channel, tile), so every
// line of u and delta is consumed by the load that fetched it (rows are
// seqlen*4 bytes apart, a power of two at the benchmark shapes, and the other
// half of a line does not survive in L2 until the next tile).  256 channels
// per workgroup, or 128+ states, fall back to 16 tokens to stay within 64 KiB
// of LDS.
template <int CPW, int NP>
struct Tile {
    static constexpr int T = (CPW >= 256 || NP >= 128) ? 16 : 32;   // tokens per tile
    static constexpr int ROW = T + 4;                 // LDS row stride (padding breaks bank aliasing)
    static constexpr int Q4 = T / 4;                  // float4 groups per tile row
};

// Sum over the LPC consecutive lanes that share a channel (lane = c*LPC + q),
// result in all of them: xor 1 and 2 (quad_perm), xor 7 within 8 lanes
// (row_half_mirror), xor 8 (row_ror:8).
template <int LPC>
__device__ __forceinline__ float LaneGroupSum(float x) {
    if constexpr (LPC >= 2) x += DppF<0xB1>(x);
    if constexpr (LPC >= 4) x += DppF<0x4E>(x);
    if constexpr (LPC >= 8) x += DppF<0x141>(x);
    if constexpr (LPC >= 16) x += DppF<0x128>(x);
    return x;
}

// FAST: seqlen % 4 == 0, 16-byte aligned rows, dim_per_group % CPW == 0 and a
// workgroup's rows under 2 GiB.
// Full tiles then move as float4 with no guards, and the one-tile-ahead
// prefetch of u/delta/B/C stays in flight through the recurrence.  A ragged
// last tile (seqlen % 32 != 0) is peeled off the loop and loaded with guards.
// Without FAST every load is guarded (clamped address + select).
template <typename IT, int LPC, int SPL, bool BVAR, bool CVAR, bool FAST>
__global__ __launch_bounds__(kThreads) void SelectiveScanFwdKernel(SelectiveScanParams p) {
    constexpr int CPW = kThreads / LPC;      // channels per workgroup
    constexpr int NP = LPC * SPL;            // padded state count
    constexpr int kTile = Tile<CPW, NP>::T;
    constexpr int kRow = Tile<CPW, NP>::ROW;
    constexpr int kQ4 = Tile<CPW, NP>::Q4;
    constexpr int ITEMS = CPW * kQ4;         // (channel, 4-token) items per tile
    constexpr int IPT = (ITEMS + kThreads - 1) / kThreads;
    constexpr int NBC = (BVAR ? 1 : 0) + (CVAR ? 1 : 0);
    constexpr int BCPT = NBC == 0 ? 1 : (NBC * NP * kQ4 + kThreads - 1) / kThreads;

    __shared__ __attribute__((aligned(16))) float sDl[CPW * kRow];        // delta' per (channel, token)
    __shared__ __attribute__((aligned(16))) float sDu[CPW * kRow];        // delta' * u
    __shared__ __attribute__((aligned(16))) float sB[BVAR ? NP * kRow : 1];
    __shared__ __attribute__((aligned(16))) float sC[CVAR ? NP * kRow : 1];
    __shared__ __attribute__((aligned(16))) float sY[CPW * kRow];         // sum over states per (channel, token)

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
    const int nvalid = FAST ? CPW : min(CPW, dpg - cb * CPW);

    const size_t row0 = (static_cast<size_t>(b) * p.dim + cbase) * static_cast<size_t>(L);
    const IT *__restrict__ ub = static_cast<const IT *>(p.u) + row0;
    const IT *__restrict__ db = static_cast<const IT *>(p.delta) + row0;
    IT *__restrict__ ob = static_cast<IT *>(p.out) + row0;
    const IT *__restrict__ Bb =
        BVAR ? static_cast<const IT *>(p.B) + (static_cast<size_t>(b) * p.groups_b + g) * static_cast<size_t>(N) * L
             : nullptr;
    const IT *__restrict__ Cb =
        CVAR ? static_cast<const IT *>(p.C) + (static_cast<size_t>(b) * p.groups_c + (BVAR ? g : 0)) * static_cast<size_t>(N) * L
             : nullptr;
    const float *const Bw = static_cast<const float *>(p.B);   // constant B/C: fp32 weights
    const float *const Cw = static_cast<const float *>(p.C);

    // ---- per-lane recurrence constants ------------------------------------
    // channel of this lane within the workgroup, and which block of SPL states
    // it holds.  With 8 lanes per channel the lanes of channel c of a wave are
    // c, c+8, ..., c+56 (the layout SwapReduce8x4 reduces over).
    // With 4 lanes per channel they are c, c+16, c+32, c+48.
    constexpr bool kSwap = LPC == 8 || LPC == 4;
    constexpr int kCpWave = 64 / LPC;    // channels per wave
    const int lane = tid & 63;
    const int lc = kSwap ? (tid >> 6) * kCpWave + lane % kCpWave : tid / LPC;
    const int lq = kSwap ? lane / kCpWave : tid % LPC;
    const bool lane_ok = lc < nvalid;
    const int dl = cbase + lc;
    float A2[SPL], h[SPL], bco[SPL], cco[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        const int n = lq * SPL + j;
        const bool ok = lane_ok && n < N;
        const size_t idx = static_cast<size_t>(dl) * N + n;
        A2[j] = ok ? p.A[idx] * kLog2eF : 0.0f;   // A_val *= kLog2e (kernel.cuh:170-178)
        bco[j] = (!BVAR && ok) ? Bw[idx] : 0.0f;
        cco[j] = (!CVAR && ok) ? Cw[idx] : 0.0f;
        if (!BVAR && !CVAR) bco[j] = bco[j] * cco[j];  // B*C folded (kernel.cuh:205-210)
        h[j] = 0.0f;
    }

    // Zero the padded state rows once; tiles only overwrite rows < N.
    if (BVAR)
        for (int i = tid; i < (NP - N) * kRow; i += kThreads) sB[N * kRow + i] = 0.0f;
    if (CVAR)
        for (int i = tid; i < (NP - N) * kRow; i += kThreads) sC[N * kRow + i] = 0.0f;

    float bias[IPT], dsk[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = tid + k * kThreads;
        const int c = it / kQ4;
        const bool ok = it < ITEMS && c < nvalid;
        bias[k] = (ok && p.delta_bias) ? p.delta_bias[cbase + c] : 0.0f;
        dsk[k] = (ok && p.D) ? p.D[cbase + c] : 0.0f;
    }

    // ---- tile loads (global -> registers) ----------------------------------
    // FAST: u, delta and y through raw-buffer descriptors over this
    // workgroup's CPW rows (under 2 GiB, checked by the host); a lane's byte
    // offset is fixed, the tile's goes in the scalar operand, so a tile costs
    // no per-lane address arithmetic.
    constexpr int EB = static_cast<int>(sizeof(IT));
    const int rows_bytes = FAST ? CPW * L * EB : 0;
    const SsRsrc ru = SsRowsRsrc(ub, rows_bytes), rdl = SsRowsRsrc(db, rows_bytes), ryo = SsRowsRsrc(ob, rows_bytes);
    int voff[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = min(tid + k * kThreads, ITEMS - 1);   // spare lanes re-read a valid item
        voff[k] = ((it / kQ4) * L + (it % kQ4) * 4) * EB;
    }
    // Two register sets of a tile's loads, used in turn by consecutive full
    // tiles, so a prefetch lands where it is consumed (no register copies).
    F4 uA[IPT], dA[IPT], bcA[BCPT], uB[IPT], dB[IPT], bcB[BCPT];
    auto load_full = [&](int t0, F4 (&ureg)[IPT], F4 (&dreg)[IPT], F4 (&bcreg)[BCPT])
                         __attribute__((always_inline)) {   // FAST, whole tile in range: no guards
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            ureg[k] = SsBufLoad4<IT>(ru, voff[k], t0 * EB);
            dreg[k] = SsBufLoad4<IT>(rdl, voff[k], t0 * EB);
        }
        if constexpr (NBC > 0) {
            const int per = N * kQ4;
#pragma unroll
            for (int k = 0; k < BCPT; ++k) {
                const int it = min(tid + k * kThreads, NBC * per - 1);
                const int r = it % per;
                const IT *row = ((BVAR && it < per) ? Bb : Cb) + static_cast<size_t>(r / kQ4) * L;
                bcreg[k] = LoadRow4Fast(row, t0 + (r % kQ4) * 4);
            }
        }
    };
    auto load_guarded = [&](int t0, F4 (&ureg)[IPT], F4 (&dreg)[IPT], F4 (&bcreg)[BCPT])
                            __attribute__((always_inline)) {   // any tile: clamped addresses, zero past the ends
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int it = tid + k * kThreads;
            const int c = min(it / kQ4, nvalid - 1), t = t0 + (it % kQ4) * 4;
            const bool ok = it < ITEMS && it / kQ4 < nvalid;
            ureg[k] = LoadRow4Guarded(ub + static_cast<size_t>(c) * L, t, L, ok);
            dreg[k] = LoadRow4Guarded(db + static_cast<size_t>(c) * L, t, L, ok);
        }
        if constexpr (NBC > 0) {
            const int per = N * kQ4;
#pragma unroll
            for (int k = 0; k < BCPT; ++k) {
                const int it = min(tid + k * kThreads, NBC * per - 1);
                const int r = it % per;
                const IT *row = ((BVAR && it < per) ? Bb : Cb) + static_cast<size_t>(r / kQ4) * L;
                bcreg[k] = LoadRow4Guarded(row, t0 + (r % kQ4) * 4, L, true);
            }
        }
    };

    // ---- phase 1: bias, softplus, delta*u into LDS; keep D*u ----------------
    F4 skip[IPT];
    auto phase1 = [&](int t0, bool full, const F4 (&ureg)[IPT], F4 (&dreg)[IPT], const F4 (&bcreg)[BCPT])
                      __attribute__((always_inline)) {
        // delta' = softplus?(delta + bias): one uniform branch per tile
        if (p.delta_softplus) {
#pragma unroll
            for (int k = 0; k < IPT; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) dreg[k].v[e] = Softplus(dreg[k].v[e] + bias[k]);
        } else {
#pragma unroll
            for (int k = 0; k < IPT; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) dreg[k].v[e] += bias[k];
        }
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int it = tid + k * kThreads;
            if (ITEMS % kThreads == 0 || it < ITEMS) {
                const int c = it / kQ4, q4 = it % kQ4;
                F4 dlv, duv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = dreg[k].v[e];
                    if (!full && t0 + q4 * 4 + e >= L) x = 0.0f;   // past the end: a = 1, b = 0
                    dlv.v[e] = x;
                    duv.v[e] = x * ureg[k].v[e];
                    skip[k].v[e] = dsk[k] * ureg[k].v[e];
                }
                *reinterpret_cast<float4 *>(&sDl[c * kRow + q4 * 4]) = make_float4(dlv.v[0], dlv.v[1], dlv.v[2], dlv.v[3]);
                *reinterpret_cast<float4 *>(&sDu[c * kRow + q4 * 4]) = make_float4(duv.v[0], duv.v[1], duv.v[2], duv.v[3]);
            }
        }
        if constexpr (NBC > 0) {
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
    };

    // ---- phase 2: the recurrence over one tile ------------------------------
    auto phase2 = [&]() __attribute__((always_inline)) {
        const float *rDl = sDl + lc * kRow;
        const float *rDu = sDu + lc * kRow;
        float *rY = sY + lc * kRow;
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
                if constexpr (BVAR) {
                    const float4 x = *reinterpret_cast<const float4 *>(sB + (lq * SPL + j) * kRow + q4 * 4);
                    bv[0] = x.x; bv[1] = x.y; bv[2] = x.z; bv[3] = x.w;
                }
                if constexpr (CVAR) {
                    const float4 x = *reinterpret_cast<const float4 *>(sC + (lq * SPL + j) * kRow + q4 * 4);
                    cv[0] = x.x; cv[1] = x.y; cv[2] = x.z; cv[3] = x.w;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = __builtin_amdgcn_exp2f(dlv[e] * A2[j]);
                    const float bt = BVAR ? bv[e] * duv[e] : duv[e];
                    h[j] = fmaf(a, h[j], bt);                 // (a1*a0, a1*b0 + b1)
                    float cc;
                    if constexpr (CVAR) cc = BVAR ? cv[e] : bco[j] * cv[e];
                    else cc = BVAR ? cco[j] : bco[j];
                    y[e] = fmaf(h[j], cc, y[e]);              // out += h * C
                }
            }
            if constexpr (LPC == 8) {
                // lanes c and c + 8 hold the same sum for the same slot: both
                // write it (no exec-mask region inside the token loop)
                rY[q4 * 4 + SwapReducedToken(lane)] = SwapReduce8x4(y);
            } else if constexpr (LPC == 4) {
                rY[q4 * 4 + SwapReducedToken(lane)] = SwapReduce4x4(y);   // every lane: a distinct (channel, token)
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[e] = LaneGroupSum<LPC>(y[e]);
                    // keep the whole reduction ahead of the branch below, so every
                    // step folds into one v_add_f32_dpp (no instruction emitted)
                    asm volatile("" : "+v"(y[e]));
                }
                if (lq == 0) *reinterpret_cast<float4 *>(rY + q4 * 4) = make_float4(y[0], y[1], y[2], y[3]);
            }
        }
    };

    // ---- phase 3: add D*u, store y -------------------------------------------
    auto phase3 = [&](int t0, bool full) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int it = tid + k * kThreads;
            const int c = it / kQ4, q4 = it % kQ4;
            if ((ITEMS % kThreads == 0 || it < ITEMS) && (FAST || c < nvalid)) {
                F4 acc = skip[k];
                const float4 x = *reinterpret_cast<const float4 *>(sY + c * kRow + q4 * 4);
                acc.v[0] += x.x; acc.v[1] += x.y; acc.v[2] += x.z; acc.v[3] += x.w;
                if (FAST && full) {
                    SsBufStore4<IT>(ryo, voff[k], t0 * EB, acc);
                } else {
                    IT *row = ob + static_cast<size_t>(c) * L;
                    StoreRow4(row, t0 + q4 * 4, L, FAST, acc);
                }
            }
        }
        // sY is rewritten only after the next phase-1 barrier; sDl/sDu/sB/sC
        // were last read before the previous barrier.
    };

    const int nfull = FAST ? L / kTile : 0;   // tiles taken on the unguarded path
    // a full tile from one register set, prefetching the next tile into the other
    auto full_tile = [&](int i, F4 (&u)[IPT], F4 (&d)[IPT], F4 (&bc)[BCPT], F4 (&nu)[IPT], F4 (&nd)[IPT],
                         F4 (&nbc)[BCPT]) __attribute__((always_inline)) {
        const int t0 = i * kTile;
        phase1(t0, true, u, d, bc);
        __syncthreads();
        if (i + 1 < nfull) load_full(t0 + kTile, nu, nd, nbc);   // prefetch; the tail tile loads after the loop
        phase2();
        __syncthreads();
        phase3(t0, true);
    };
    if (nfull > 0) {   // the only path into the full-tile loop
        load_full(0, uA, dA, bcA);
        // A tile is entered with its loads issued before the previous tile's
        // IPT stores (vmcnt counts both).  Dropped stores (beyond the
        // descriptor) after tile 0's loads give the first entry the same
        // order, so the loop head's wait lets the stores run on; with the loads
        // alone on that path (or the guarded path of nfull = 0 merging into
        // it) it waited for every store to complete.  Interleaved A/B: 8 x
        // 5120 x 2048 0.3407 -> 0.3343 ms, 2 x 4096 x 4096 0.2225 -> 0.2131,
        // 4 x 5120 x 2048 0.2045 -> 0.2016 (an unconditional prefetch on top,
        // the last tile reloaded: 0.3323, 0.2295, 0.2012).
#pragma unroll
        for (int k = 0; k < IPT; ++k) SsBufStore4<IT>(ryo, kSsDropOffset, 0, F4{});
        for (int i = 0;; i += 2) {
            full_tile(i, uA, dA, bcA, uB, dB, bcB);
            if (i + 1 >= nfull) break;
            full_tile(i + 1, uB, dB, bcB, uA, dA, bcA);
            if (i + 2 >= nfull) break;
        }
    }
    for (int t0 = nfull * kTile; t0 < L; t0 += kTile) {   // ragged tail (FAST) or every tile
        load_guarded(t0, uA, dA, bcA);
        phase1(t0, false, uA, dA, bcA);
        __syncthreads();
        phase2();
        __syncthreads();
        phase3(t0, false);
    }
    // Scan state after the last token (tokens past the end kept it unchanged).
    if (p.last_state != nullptr && lane_ok) {
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const int n = lq * SPL + j;
            if (n < N) p.last_state[(static_cast<size_t>(b) * p.dim + dl) * N + n] = h[j];
        }
    }
}

struct Config {
    int lpc, spl;
};

// States per lane and lanes per channel by dstate.  The ss_lpc override sets
// the lanes per channel for dstate <= 16 (1, 2, 4, 8 or 16), for tests and tuning.
Config ChooseConfig(int N) {
    if (N <= 16) {
        const int forced = static_cast<int>(GetOverride(kOverrideSsLpc));
        switch (forced) {
            case 4: if (N > 8) return {4, 4}; break;
            case 8: return {8, 2};
            case 16: return {16, 1};
            case 2: if (N <= 8) return {2, 4}; break;
            case 1: if (N <= 4) return {1, 4}; break;
            default: break;
        }
        if (N <= 4) return {1, 4};
        if (N <= 8) return {2, 4};
        return {8, 2};   // measured: 0.445 ms vs 0.454 ms (4 lanes) at 8 x 5120 x 2048 x 16
    }
    if (N <= 32) return {8, 4};
    if (N <= 64) return {16, 4};
    if (N <= 128) return {16, 8};
    return {16, 16};
}

template <typename IT, int LPC, int SPL, bool BVAR, bool CVAR, bool VEC>
void NoteSs() {
    XM_NOTE_LAUNCH("SelectiveScanFwdKernel", {TypeTag<IT>()}, LPC, SPL, BVAR, CVAR, VEC);
}

template <typename IT, int LPC, int SPL, bool VEC>
void LaunchLSV(const SelectiveScanParams &p, dim3 grid, hipStream_t stream) {
    if (p.b_var && p.c_var) NoteSs<IT, LPC, SPL, true, true, VEC>();
    else if (p.b_var) NoteSs<IT, LPC, SPL, true, false, VEC>();
    else if (p.c_var) NoteSs<IT, LPC, SPL, false, true, VEC>();
    else NoteSs<IT, LPC, SPL, false, false, VEC>();
    if (p.b_var && p.c_var)
        hipLaunchKernelGGL((SelectiveScanFwdKernel<IT, LPC, SPL, true, true, VEC>), grid, dim3(kThreads), 0, stream, p);
    else if (p.b_var)
        hipLaunchKernelGGL((SelectiveScanFwdKernel<IT, LPC, SPL, true, false, VEC>), grid, dim3(kThreads), 0, stream, p);
    else if (p.c_var)
        hipLaunchKernelGGL((SelectiveScanFwdKernel<IT, LPC, SPL, false, true, VEC>), grid, dim3(kThreads), 0, stream, p);
    else
        hipLaunchKernelGGL((SelectiveScanFwdKernel<IT, LPC, SPL, false, false, VEC>), grid, dim3(kThreads), 0, stream, p);
}

template <typename IT, int LPC, int SPL>
void LaunchLS(const SelectiveScanParams &p, int vec, dim3 grid, hipStream_t stream) {
    constexpr int CPW = kThreads / LPC;
    // the fast path's row descriptors span a workgroup's CPW rows: under 2 GiB
    const bool rows_fit = static_cast<long long>(CPW) * p.seqlen * static_cast<long long>(sizeof(IT)) < (1LL << 31);
    if (vec && rows_fit && p.dim_per_group % CPW == 0) LaunchLSV<IT, LPC, SPL, true>(p, grid, stream);
    else LaunchLSV<IT, LPC, SPL, false>(p, grid, stream);
}

// vector accesses are 4 elements: 16 bytes of fp32, 8 of 16-bit data
bool AlignedVec(const void *ptr, int elem_bytes) {
    return (reinterpret_cast<uintptr_t>(ptr) & static_cast<uintptr_t>(4 * elem_bytes - 1)) == 0;
}

template <typename IT>
void LaunchTyped(const SelectiveScanParams &p, const Config &cfg, dim3 grid, hipStream_t stream) {
    const int eb = static_cast<int>(sizeof(IT));
    const int vec = (p.seqlen % 4 == 0) && AlignedVec(p.u, eb) && AlignedVec(p.delta, eb) && AlignedVec(p.out, eb) &&
                    (!p.b_var || AlignedVec(p.B, eb)) && (!p.c_var || AlignedVec(p.C, eb));
    switch (cfg.lpc * 100 + cfg.spl) {
        case 104: LaunchLS<IT, 1, 4>(p, vec, grid, stream); break;
        case 204: LaunchLS<IT, 2, 4>(p, vec, grid, stream); break;
        case 404: LaunchLS<IT, 4, 4>(p, vec, grid, stream); break;
        case 802: LaunchLS<IT, 8, 2>(p, vec, grid, stream); break;
        case 1601: LaunchLS<IT, 16, 1>(p, vec, grid, stream); break;
        case 804: LaunchLS<IT, 8, 4>(p, vec, grid, stream); break;
        case 1604: LaunchLS<IT, 16, 4>(p, vec, grid, stream); break;
        case 1608: LaunchLS<IT, 16, 8>(p, vec, grid, stream); break;
        default: LaunchLS<IT, 16, 16>(p, vec, grid, stream); break;
    }
}

// d_state = 0: no state, y = D * u (zeros without D); reference
// selective_scan_fwd_kernel.cuh:161 (out = D * u) with an empty state loop (:166).
template <typename IT>
__global__ __launch_bounds__(256) void SelectiveScanSkipKernel(SelectiveScanParams p) {
    const size_t total = static_cast<size_t>(p.batch) * p.dim * p.seqlen;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    const IT *u = static_cast<const IT *>(p.u);
    IT *out = static_cast<IT *>(p.out);
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int d = static_cast<int>((i / static_cast<size_t>(p.seqlen)) % static_cast<size_t>(p.dim));
        const float dv = p.D != nullptr ? p.D[d] : 0.0f;
        out[i] = FromF<IT>(dv * ToF(u[i]));
    }
}

template <typename IT>
void LaunchSkip(const SelectiveScanParams &p, hipStream_t stream) {
    const size_t total = static_cast<size_t>(p.batch) * p.dim * p.seqlen;
    const size_t blocks = std::min<size_t>((total + 255) / 256, 8192);
    XM_NOTE_LAUNCH("SelectiveScanSkipKernel", {TypeTag<IT>()}, );
    hipLaunchKernelGGL(SelectiveScanSkipKernel<IT>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
}

}  // namespace

void LaunchSelectiveScan(const SelectiveScanParams &p, void *stream_v) {
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    if (p.dstate == 0) {
        if (p.in_type == XM_ELEM_FLOAT16) LaunchSkip<_Float16>(p, stream);
        else if (p.in_type == XM_ELEM_BFLOAT16) LaunchSkip<Bf16>(p, stream);
        else LaunchSkip<float>(p, stream);
        XM_LAUNCH_CHECK("SelectiveScanFn (d_state 0)");
        return;
    }
    const Config cfg = ChooseConfig(p.dstate);
    const int cpw = kThreads / cfg.lpc;
    const long long ncb = (p.dim_per_group + cpw - 1) / cpw;
    const long long blocks = ncb * p.groups_b * static_cast<long long>(p.batch);
    // Fewer channel blocks than CUs and a sequence long enough to split: scan
    // segments of the sequence in parallel, one workgroup per channel
    // (ss_split override: 1 keeps the channel blocks, 2 always splits).
    const int64_t split = GetOverride(kOverrideSsSplit);
    if (SelectiveScanSegFits(p) &&
        (split == 2 || (split == 0 && blocks < kSegMaxChannelBlocks && p.seqlen >= kSegMinSeqlen))) {
        LaunchSelectiveScanSeg(p, stream);
        return;
    }
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "SelectiveScanFn launch exceeds the grid limit");
    const dim3 grid(static_cast<unsigned>(blocks));
    if (p.in_type == XM_ELEM_FLOAT16) LaunchTyped<_Float16>(p, cfg, grid, stream);
    else if (p.in_type == XM_ELEM_BFLOAT16) LaunchTyped<Bf16>(p, cfg, grid, stream);
    else LaunchTyped<float>(p, cfg, grid, stream);
    XM_LAUNCH_CHECK("SelectiveScanFn");
}

}  // namespace xm
