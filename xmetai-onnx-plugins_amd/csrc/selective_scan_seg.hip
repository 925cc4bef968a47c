// SelectiveScanFn forward, sequence-parallel form (gfx950, wave64).
//
// The single-pass kernel (selective_scan.hip) gives each channel one chain of
// seqlen dependent steps and fills the chip only when batch x channels
// supplies hundreds of workgroups.  With few channels (a short batch, a small
// layer, a long sequence) most CUs sit idle while a handful walk the whole
// sequence.  This kernel scans the sequence in parallel instead.
//
// The recurrence h_t = a_t h_{t-1} + b_t (a_t = exp2(delta'_t A2), b_t =
// B_t delta'_t u_t) is one affine map per token, and maps compose
// associatively, (a2, b2) o (a1, b1) = (a2 a1, a2 b1 + b2): the reference's
// SSMScanOp (selective_scan_common.h:148-153), whose block prefix it carries
// from chunk to chunk (SSMScanPrefixCallbackOp, :170-182;
// selective_scan_fwd_kernel.cuh:239-257).
//
// A workgroup owns one channel (b, d) and cuts each block of LB = S x 16
// tokens into S = NWV x SW segments of 16 tokens, SW = 64 / LPC per wave.
// Lane = q * SW + s: q is the lane's block of SPL states, s its segment in the
// wave, so a segment's state lanes are SW lanes apart and the segments of a
// state block are adjacent lanes.  Per block:
//  1. stage delta' = softplus?(delta + bias), delta' u and D u in LDS with
//     coalesced loads (and store the previous block's y);
//  2. pass 1: every lane runs its segment from a zero state, giving the map
//     (P, H) of the segment per state: H the end state, P = exp2(A2 sum
//     delta'); with at most two states per lane the decays, the inputs and
//     the C rows stay in registers for pass 2, otherwise pass 2 reloads them;
//  3. combine: a Kogge-Stone scan with DPP row_shr 1/2/4/8 composes the maps
//     over the segments of a wave, the wave totals meet in LDS, the block's
//     carry (the state before its first token, held in VGPRs) is the first
//     map, and a row_shr:1 move turns each lane's inclusive map into its
//     segment's start state;
//  4. pass 2: every lane reruns its segment from that state, accumulating
//     C_t h_t over its states; lane swaps add the state lanes of a segment.
// The block's end state becomes the next block's carry in every lane.  The
// arithmetic is about 1.3x (two states per lane) to 1.8x (more) that of the
// single pass, traded for S-fold shorter dependent chains and one workgroup
// per channel.
//
// B/C rows come through raw buffer loads: tokens past the sequence and
// padded states read zeros with no branch, so padding tokens are identity
// maps (delta' = 0 gives a = 1, b = 0).  z is never read (output 0 does not
// depend on it, selective_scan_fwd_kernel.cuh:280 vs :296-299).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "selective_scan_dev.h"
#include "xm_hip.h"
#include "xm_matrix.h"
#include "xm_params.h"

namespace xm {
namespace {

using namespace ssdev;

constexpr int kSegLen = 16;              // tokens per segment
constexpr int kSegGroups = kSegLen / 4;  // four-token groups per segment
constexpr int kSegRow = kSegLen + 4;     // LDS stride of a segment (padding against bank aliasing)
constexpr int kSegWaves = 4;             // waves per workgroup

// DPP move within a row of 16 lanes; lanes whose source lies outside the row
// keep `old`.
template <int CTRL>
__device__ __forceinline__ float RowMove(float old, float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// One Kogge-Stone step: lanes with `take` put the map of the lane K below
// (earlier segments) before their own.
template <int K>
__device__ __forceinline__ void ScanStep(float &P, float &H, bool take) {
    const float pp = RowMove<0x110 + K>(1.0f, P);   // row_shr:K
    const float hp = RowMove<0x110 + K>(0.0f, H);
    const float nh = fmaf(P, hp, H);
    const float np = P * pp;
    H = take ? nh : H;
    P = take ? np : P;
}

// Inclusive scan of the maps over the SW adjacent segment lanes (SW <= 16,
// groups aligned inside DPP rows): afterwards lane s holds segments 0..s
// composed.
template <int SW>
__device__ __forceinline__ void SegScanInclusive(float &P, float &H, int s) {
    static_assert(SW >= 2 && SW <= 16, "segments of a state block share one DPP row");
    ScanStep<1>(P, H, s >= 1);
    if constexpr (SW > 2) ScanStep<2>(P, H, s >= 2);
    if constexpr (SW > 4) ScanStep<4>(P, H, s >= 4);
    if constexpr (SW > 8) ScanStep<8>(P, H, s >= 8);
}

// Inclusive -> exclusive: the map of segments 0..s-1 (identity for s = 0).
__device__ __forceinline__ void SegScanShift(float &P, float &H, int s) {
    const float pp = RowMove<0x111>(1.0f, P);   // row_shr:1
    const float hp = RowMove<0x111>(0.0f, H);
    P = s == 0 ? 1.0f : pp;
    H = s == 0 ? 0.0f : hp;
}

// Sum of y[0..3] over the LPC state lanes of a segment (lanes SW apart).  On
// return lane l holds the sum for segment l % SW and token {0, 2, 1, 3}[l / 16].
template <int LPC>
__device__ __forceinline__ float SegStateSum(const float (&y)[4]) {
    if constexpr (LPC == 8) {
        return SwapReduce8x4(y);
    } else {
        float z = SwapReduce4x4(y);                           // lanes 16 apart
        if constexpr (LPC == 16) {
            z += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(z), 0x124, 0xf, 0xf, true));   // row_ror:4
            z += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(z), 0x128, 0xf, 0xf, true));   // row_ror:8
        }
        return z;
    }
}

__device__ __forceinline__ Rsrc RowsRsrc(const void *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), bytes, kRawBufferWord3);
}

// Tokens t..t+3 of the B/C row that starts at element `roff` (-1: a padded
// state), zeros past the sequence end.  VEC: seqlen % 4 == 0 and aligned
// rows, so a group is entirely inside or outside the sequence.
template <typename IT, bool VEC>
__device__ __forceinline__ F4 BufRow4(Rsrc r, int roff, int t, int L) {
    constexpr int EB = static_cast<int>(sizeof(IT));
    F4 o;
    if constexpr (VEC) {
        const int off = (roff >= 0 && t < L) ? (roff + t) * EB : kOutOfRange;
        if constexpr (EB == 4) {
            const v4f x = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
            o = F4{{x[0], x[1], x[2], x[3]}};
        } else {
            const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
            if constexpr (std::is_same_v<IT, _Float16>) {
                const h4 hv = __builtin_bit_cast(h4, x);
                o = F4{{static_cast<float>(hv[0]), static_cast<float>(hv[1]), static_cast<float>(hv[2]),
                        static_cast<float>(hv[3])}};
            } else {
                o = F4{{__uint_as_float(x.x << 16), __uint_as_float(x.x & 0xffff0000u), __uint_as_float(x.y << 16),
                        __uint_as_float(x.y & 0xffff0000u)}};
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int off = (roff >= 0 && t + e < L) ? (roff + t + e) * EB : kOutOfRange;
            if constexpr (EB == 4) {
                o.v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
            } else {
                const unsigned short bits = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
                if constexpr (std::is_same_v<IT, _Float16>) o.v[e] = static_cast<float>(__builtin_bit_cast(_Float16, bits));
                else o.v[e] = __uint_as_float(static_cast<uint32_t>(bits) << 16);
            }
        }
    }
    return o;
}

template <typename IT, int LPC, int SPL, bool BVAR, bool CVAR, bool VEC>
__global__ __launch_bounds__(64 * kSegWaves) void SelectiveScanSegKernel(SelectiveScanParams p) {
    constexpr int NT = 64 * kSegWaves;
    constexpr int SW = 64 / LPC;             // segments per wave
    constexpr int S = kSegWaves * SW;        // segments per block
    constexpr int LB = S * kSegLen;          // tokens per block
    constexpr int NP = LPC * SPL;            // padded state count
    constexpr int ITEMS = LB / 4;            // four-token items staged per block
    constexpr int IPT = (ITEMS + NT - 1) / NT;
    constexpr bool KEEP = SPL <= 2;          // pass-1 decays and inputs reused by pass 2

    __shared__ __attribute__((aligned(16))) float sDl[S * kSegRow];   // delta'
    __shared__ __attribute__((aligned(16))) float sDu[S * kSegRow];   // delta' * u
    __shared__ __attribute__((aligned(16))) float sSk[S * kSegRow];   // D * u
    __shared__ __attribute__((aligned(16))) float sY[S * kSegRow];    // sum over states of C h
    __shared__ float sTp[kSegWaves][NP], sTh[kSegWaves][NP];          // wave totals (P, H) per state

    const int L = p.seqlen;
    const int N = p.dstate;
    // Consecutive channels of one batch row share its B/C rows: keep them on one XCD's L2.
    const int x = XcdLocalBlock(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
    const int d = x % p.dim;
    const int b = x / p.dim;
    const int g = d / p.dim_per_group;

    const size_t row = (static_cast<size_t>(b) * p.dim + d) * static_cast<size_t>(L);
    const IT *__restrict__ urow = static_cast<const IT *>(p.u) + row;
    const IT *__restrict__ drow = static_cast<const IT *>(p.delta) + row;
    IT *__restrict__ orow = static_cast<IT *>(p.out) + row;
    const size_t nl = static_cast<size_t>(N) * L;
    const int nl_bytes = static_cast<int>(nl * sizeof(IT));          // < 2^31, checked by the launcher
    const Rsrc rB = RowsRsrc(BVAR ? static_cast<const IT *>(p.B) + (static_cast<size_t>(b) * p.groups_b + g) * nl
                                  : p.B, BVAR ? nl_bytes : 0);
    const Rsrc rC = RowsRsrc(CVAR ? static_cast<const IT *>(p.C) +
                                        (static_cast<size_t>(b) * p.groups_c + (BVAR ? g : 0)) * nl
                                  : p.C, CVAR ? nl_bytes : 0);

    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int lane = tid & 63;
    const int q = lane / SW;
    const int s = lane % SW;
    const int seg = w * SW + s;
    const int sbase = seg * kSegRow;

    // Per-state constants (reference selective_scan_fwd_kernel.cuh:170-210):
    // A in log2 units; constant B and C folded into the readout weight.
    float A2[SPL], bco[SPL], cco[SPL], cb[SPL];
    int roff[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        const int n = q * SPL + j;
        const bool ok = n < N;
        const size_t idx = static_cast<size_t>(d) * N + n;
        A2[j] = ok ? p.A[idx] * kLog2eF : 0.0f;
        bco[j] = (!BVAR && ok) ? static_cast<const float *>(p.B)[idx] : 0.0f;
        cco[j] = (!CVAR && ok) ? static_cast<const float *>(p.C)[idx] : 0.0f;
        if (!BVAR && !CVAR) bco[j] = bco[j] * cco[j];
        roff[j] = ok ? n * L : -1;
        cb[j] = 0.0f;   // the state before the first token
    }
    const float bias = p.delta_bias != nullptr ? p.delta_bias[d] : 0.0f;
    const float dsk = p.D != nullptr ? p.D[d] : 0.0f;

    // ---- 1. stage a block (and store the block before it) ---------------------
    auto stage = [&](int t0, bool store_prev) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int i = tid + k * NT;
            if (ITEMS % NT == 0 || i < ITEMS) {
                const int li = (i >> 2) * kSegRow + (i & 3) * 4;   // segment i/4, group i%4
                const int t = t0 + 4 * i;
                if (store_prev) {   // every token of the previous block lies before t0 < L
                    const float4 yv = *reinterpret_cast<const float4 *>(&sY[li]);
                    const float4 kv = *reinterpret_cast<const float4 *>(&sSk[li]);
                    const F4 o{{kv.x + yv.x, kv.y + yv.y, kv.z + yv.z, kv.w + yv.w}};
                    if constexpr (VEC) StoreRow4Fast(orow, t - LB, o);
                    else StoreRow4(orow, t - LB, L, false, o);
                }
                F4 uu, dd;
                if (VEC && t + 3 < L) {
                    uu = LoadRow4Fast(urow, t);
                    dd = LoadRow4Fast(drow, t);
                } else {
                    uu = LoadRow4Guarded(urow, t, L, true);
                    dd = LoadRow4Guarded(drow, t, L, true);
                }
                F4 dl, du, sk;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = dd.v[e] + bias;
                    if (p.delta_softplus) v = Softplus(v);
                    v = t + e < L ? v : 0.0f;   // past the end: a = 1, b = 0
                    dl.v[e] = v;
                    du.v[e] = v * uu.v[e];
                    sk.v[e] = dsk * uu.v[e];
                }
                *reinterpret_cast<float4 *>(&sDl[li]) = make_float4(dl.v[0], dl.v[1], dl.v[2], dl.v[3]);
                *reinterpret_cast<float4 *>(&sDu[li]) = make_float4(du.v[0], du.v[1], du.v[2], du.v[3]);
                *reinterpret_cast<float4 *>(&sSk[li]) = make_float4(sk.v[0], sk.v[1], sk.v[2], sk.v[3]);
            }
        }
    };

    const int nblocks = (L + LB - 1) / LB;
    for (int blk = 0; blk < nblocks; ++blk) {
        const int t0 = blk * LB;
        const int ts = t0 + seg * kSegLen;   // this lane's first token
        stage(t0, blk > 0);
        __syncthreads();

        // ---- 2. pass 1: the segment's map from a zero state ----------------------
        // B rows: the whole segment up front at two states per lane, else per group
        F4 bq[kSegGroups][SPL];
        if constexpr (BVAR && KEEP) {
#pragma unroll
            for (int gi = 0; gi < kSegGroups; ++gi)
#pragma unroll
                for (int j = 0; j < SPL; ++j) bq[gi][j] = BufRow4<IT, VEC>(rB, roff[j], ts + 4 * gi, L);
        }
        float ka[KEEP ? kSegGroups : 1][SPL][4], kb[KEEP ? kSegGroups : 1][SPL][4];
        float P[SPL], H[SPL];
        float sdl = 0.0f;
#pragma unroll
        for (int j = 0; j < SPL; ++j) H[j] = 0.0f;
#pragma unroll
        for (int gi = 0; gi < kSegGroups; ++gi) {
            const float4 dl4 = *reinterpret_cast<const float4 *>(&sDl[sbase + 4 * gi]);
            const float4 du4 = *reinterpret_cast<const float4 *>(&sDu[sbase + 4 * gi]);
            const float dl[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
            const float du[4] = {du4.x, du4.y, du4.z, du4.w};
            if constexpr (BVAR && !KEEP) {
#pragma unroll
                for (int j = 0; j < SPL; ++j) bq[gi][j] = BufRow4<IT, VEC>(rB, roff[j], ts + 4 * gi, L);
            }
#pragma unroll
            for (int j = 0; j < SPL; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = __builtin_amdgcn_exp2f(dl[e] * A2[j]);
                    const float bt = BVAR ? bq[gi][j].v[e] * du[e] : du[e];
                    H[j] = fmaf(a, H[j], bt);
                    if constexpr (KEEP) {
                        ka[gi][j][e] = a;
                        kb[gi][j][e] = bt;
                    }
                }
            sdl += (dl[0] + dl[1]) + (dl[2] + dl[3]);
        }
#pragma unroll
        for (int j = 0; j < SPL; ++j) P[j] = __builtin_amdgcn_exp2f(sdl * A2[j]);   // prod of the decays

        // C rows for pass 2 at two states per lane, in flight through the combine
        F4 cq[kSegGroups][SPL];
        if constexpr (CVAR && KEEP) {
#pragma unroll
            for (int gi = 0; gi < kSegGroups; ++gi)
#pragma unroll
                for (int j = 0; j < SPL; ++j) cq[gi][j] = BufRow4<IT, VEC>(rC, roff[j], ts + 4 * gi, L);
        }

        // ---- 3. combine: segment scan in the wave, wave totals across the block ----
#pragma unroll
        for (int j = 0; j < SPL; ++j) SegScanInclusive<SW>(P[j], H[j], s);
        if (s == SW - 1) {
#pragma unroll
            for (int j = 0; j < SPL; ++j) {
                sTp[w][q * SPL + j] = P[j];
                sTh[w][q * SPL + j] = H[j];
            }
        }
#pragma unroll
        for (int j = 0; j < SPL; ++j) SegScanShift(P[j], H[j], s);
        __syncthreads();
        float h[SPL];
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const int n = q * SPL + j;
            float c = cb[j], start = 0.0f;
#pragma unroll
            for (int v = 0; v < kSegWaves; ++v) {
                start = v == w ? c : start;          // the state before wave v's first segment
                c = fmaf(sTp[v][n], c, sTh[v][n]);
            }
            cb[j] = c;                               // the state after this block
            h[j] = fmaf(P[j], start, H[j]);          // the state before this lane's segment
        }

        // ---- 4. pass 2: the segment from its start state, y_t = sum_n C h ---------
#pragma unroll
        for (int gi = 0; gi < kSegGroups; ++gi) {
            float dl[4], du[4];
            if constexpr (!KEEP) {
                const float4 dl4 = *reinterpret_cast<const float4 *>(&sDl[sbase + 4 * gi]);
                const float4 du4 = *reinterpret_cast<const float4 *>(&sDu[sbase + 4 * gi]);
                dl[0] = dl4.x; dl[1] = dl4.y; dl[2] = dl4.z; dl[3] = dl4.w;
                du[0] = du4.x; du[1] = du4.y; du[2] = du4.z; du[3] = du4.w;
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    if constexpr (BVAR) bq[gi][j] = BufRow4<IT, VEC>(rB, roff[j], ts + 4 * gi, L);
                    if constexpr (CVAR) cq[gi][j] = BufRow4<IT, VEC>(rC, roff[j], ts + 4 * gi, L);
                }
            }
            float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < SPL; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float a, bt;
                    if constexpr (KEEP) {
                        a = ka[gi][j][e];
                        bt = kb[gi][j][e];
                    } else {
                        a = __builtin_amdgcn_exp2f(dl[e] * A2[j]);
                        bt = BVAR ? bq[gi][j].v[e] * du[e] : du[e];
                    }
                    h[j] = fmaf(a, h[j], bt);
                    float cc;
                    if constexpr (CVAR) cc = BVAR ? cq[gi][j].v[e] : bco[j] * cq[gi][j].v[e];
                    else cc = BVAR ? cco[j] : bco[j];
                    y[e] = fmaf(h[j], cc, y[e]);
                }
            float z = SegStateSum<LPC>(y);
            asm volatile("" : "+v"(z));   // keep the whole reduction ahead of the branch
            if ((lane & 15) < SW) sY[sbase + 4 * gi + SwapReducedToken(lane)] = z;
        }
        __syncthreads();
    }

    // ---- the last block's y ---------------------------------------------------------
    {
        const int t0 = (nblocks - 1) * LB;
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int i = tid + k * NT;
            const int t = t0 + 4 * i;
            if ((ITEMS % NT == 0 || i < ITEMS) && t < L) {
                const int li = (i >> 2) * kSegRow + (i & 3) * 4;
                const float4 yv = *reinterpret_cast<const float4 *>(&sY[li]);
                const float4 kv = *reinterpret_cast<const float4 *>(&sSk[li]);
                const F4 o{{kv.x + yv.x, kv.y + yv.y, kv.z + yv.z, kv.w + yv.w}};
                StoreRow4(orow, t, L, VEC, o);
            }
        }
    }
    // Scan state after the last token (padding tokens are identity maps).
    if (p.last_state != nullptr && s == 0) {
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const int n = q * SPL + j;
            if (n < N) p.last_state[(static_cast<size_t>(b) * p.dim + d) * N + n] = cb[j];
        }
    }
}

struct SegConfig {
    int lpc, spl;
};

// Lanes per segment and states per lane by dstate: two states per lane up to
// 32 states (pass 1's decays kept in registers), then 4, 8, 16.
SegConfig ChooseSegConfig(int N) {
    if (N <= 4) return {4, 1};
    if (N <= 8) return {8, 1};
    if (N <= 16) return {8, 2};
    if (N <= 32) return {16, 2};
    if (N <= 64) return {16, 4};
    if (N <= 128) return {16, 8};
    return {16, 16};
}

template <typename IT, int LPC, int SPL, bool BVAR, bool CVAR, bool VEC>
void LaunchSeg(const SelectiveScanParams &p, dim3 grid, hipStream_t stream) {
    XM_NOTE_LAUNCH("SelectiveScanSegKernel", {TypeTag<IT>()}, LPC, SPL, BVAR, CVAR, VEC);
    hipLaunchKernelGGL((SelectiveScanSegKernel<IT, LPC, SPL, BVAR, CVAR, VEC>), grid, dim3(64 * kSegWaves), 0, stream,
                       p);
}

template <typename IT, int LPC, int SPL, bool VEC>
void LaunchSegLSV(const SelectiveScanParams &p, dim3 grid, hipStream_t stream) {
    if (p.b_var && p.c_var) LaunchSeg<IT, LPC, SPL, true, true, VEC>(p, grid, stream);
    else if (p.b_var) LaunchSeg<IT, LPC, SPL, true, false, VEC>(p, grid, stream);
    else if (p.c_var) LaunchSeg<IT, LPC, SPL, false, true, VEC>(p, grid, stream);
    else LaunchSeg<IT, LPC, SPL, false, false, VEC>(p, grid, stream);
}

template <typename IT, int LPC, int SPL>
void LaunchSegLS(const SelectiveScanParams &p, bool vec, dim3 grid, hipStream_t stream) {
    if (vec) LaunchSegLSV<IT, LPC, SPL, true>(p, grid, stream);
    else LaunchSegLSV<IT, LPC, SPL, false>(p, grid, stream);
}

bool Aligned4(const void *ptr, int elem_bytes) {
    return (reinterpret_cast<uintptr_t>(ptr) & static_cast<uintptr_t>(4 * elem_bytes - 1)) == 0;
}

template <typename IT>
void LaunchSegTyped(const SelectiveScanParams &p, dim3 grid, hipStream_t stream) {
    const int eb = static_cast<int>(sizeof(IT));
    const bool vec = (p.seqlen % 4 == 0) && Aligned4(p.u, eb) && Aligned4(p.delta, eb) && Aligned4(p.out, eb) &&
                     (!p.b_var || Aligned4(p.B, eb)) && (!p.c_var || Aligned4(p.C, eb));
    const SegConfig cfg = ChooseSegConfig(p.dstate);
    switch (cfg.lpc * 100 + cfg.spl) {
        case 401: LaunchSegLS<IT, 4, 1>(p, vec, grid, stream); break;
        case 801: LaunchSegLS<IT, 8, 1>(p, vec, grid, stream); break;
        case 802: LaunchSegLS<IT, 8, 2>(p, vec, grid, stream); break;
        case 1602: LaunchSegLS<IT, 16, 2>(p, vec, grid, stream); break;
        case 1604: LaunchSegLS<IT, 16, 4>(p, vec, grid, stream); break;
        case 1608: LaunchSegLS<IT, 16, 8>(p, vec, grid, stream); break;
        default: LaunchSegLS<IT, 16, 16>(p, vec, grid, stream); break;
    }
}

}  // namespace

bool SelectiveScanSegFits(const SelectiveScanParams &p) {
    const size_t elem = p.in_type == XM_ELEM_FLOAT ? 4 : 2;
    const size_t rows = static_cast<size_t>(p.dstate) * static_cast<size_t>(p.seqlen) * elem;
    const size_t channels = static_cast<size_t>(p.batch) * static_cast<size_t>(p.dim);
    return p.dstate >= 1 && p.dstate <= 256 && rows < (size_t{1} << 31) && channels <= 2147483647u;
}

void LaunchSelectiveScanSeg(const SelectiveScanParams &p, void *stream_v) {
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    if (!SelectiveScanSegFits(p)) throw Error(XM_ERR_UNSUPPORTED, "SelectiveScanFn sequence-split form does not fit");
    const dim3 grid(static_cast<unsigned>(static_cast<size_t>(p.batch) * p.dim));
    if (p.in_type == XM_ELEM_FLOAT16) LaunchSegTyped<_Float16>(p, grid, stream);
    else if (p.in_type == XM_ELEM_BFLOAT16) LaunchSegTyped<Bf16>(p, grid, stream);
    else LaunchSegTyped<float>(p, grid, stream);
    XM_LAUNCH_CHECK("SelectiveScanFn (sequence split)");
}

}  // namespace xm
