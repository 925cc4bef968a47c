// Mamba3SisoFn forward for gfx950 (CDNA4, wave64).
//
// Math (reference mamba3_siso_fwd.cu:79-171), per (b,h) with state S [P,N]
// and angle state theta [A], for t = 0..T-1:
//   theta = wrap(theta + tanh(Angles_t) * DT_t * pi)            (wrap to [0, 2pi))
//   q = Q_t + Q_bias, k = K_t + K_bias, qk = q.k (unrotated)
//   rotate pairs p < A of q and k by theta_p
//   gamma = DT_t sigmoid(Trap_t); look = DT_{t+1} (1 - sigmoid(Trap_{t+1})) (0 at t = T-1)
//   S *= exp(ADT_t);  y = q_rot.S + (D + qk gamma) V_t  (* silu(Z_t));  S += V_t (x) k_rot (gamma + look)
//
// One fused kernel.  A workgroup of 512 threads owns one (b,h) and 32 state
// rows (P), so the usual P = 64 takes two workgroups per head and a 4 x 32
// head workload fills the 256 CUs with one workgroup each.  The sequence is
// walked in blocks of TB tokens; the per-token vectors of block j+1 are
// prepared while block j's recurrence runs, in double-buffered LDS, with two
// barriers per block:
//   prep A (per wave: SEG = TB/8 consecutive tokens x every pair): angle
//     increments tanh(Angles) * DT * pi in fp64 and their running sum over
//     the wave's tokens;
//   prep B: each wave adds the block carry and the sums of the earlier waves,
//     wraps with the reference's period 2 * (float)pi, rotates q/k with the
//     hardware sine/cosine of the wrapped angle (v_sin/v_cos take revolutions;
//     the revolutions are formed in fp64), writes rotated q and k to LDS, sums
//     q.k over the pairs, and one lane per token forms decay, gamma + look and
//     the diagonal D + qk gamma;
//   recurrence: lane (row group rg, key group kg) holds KPT keys of one row
//     of S in VGPRs; the readout over keys is a 4-step DPP row sum; token
//     tt+1's vectors are read from LDS while token tt computes; lane kg keeps
//     the output of tokens kg and kg+16 and stores them after the block.
// Summing the angle increments first and wrapping once per token equals the
// reference's wrap after every step in exact arithmetic; fp64 keeps the
// difference far below fp32 resolution.  Pairs >= A are not rotated (:109).
// Tokens past the end of the last block are identity tokens (decay 1, zero
// k scale, zero v): they leave the state unchanged and are not stored.
//
// States (a widening; the reference rejects has_input_states and
// return_final_states, mamba3_siso_fn_ort.cpp:50-55): (ssm [P,N], angle [A],
// k [N], v [P]) per (b,h).  The final ones are S and theta after the last
// token (whose look-ahead is 0), its rotated k and its V; given as input they
// start the scan from S = ssm + v (x) k * DT_0 (1 - sigmoid(Trap_0)), the
// last token's look-ahead now that its successor is known, and theta = angle,
// so two calls chained through the states equal one call.
//
// Packed sequences (cu_seqlens, a widening): batch indexes sequences packed
// along one row of seqlen tokens; a workgroup reads its sequence's offsets
// (clamped into [0, seqlen]; an inverted range is empty, and an empty
// sequence passes its states through, its pending look-ahead included).
//
// headdim_qk above 512 (KB): the keys are taken in blocks of at most 512, one
// launch each.  A key's state column, its rotation pair and angle, and its
// state inputs and outputs depend on no other key; the readout q.S and the
// unrotated q.k are sums over keys.  So each launch runs the recurrence on its
// block's keys and adds its part of y to what the earlier launches wrote; the
// first adds D v, the last applies the Z gate.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "mamba3_math.h"
#include "xm_hip.h"
#include "xm_params.h"

namespace xm {
namespace {

using namespace m3;

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = kThreads / 16;     // state rows per workgroup (one per 16-lane row group)

template <int KPT>
struct M3Layout {
    static constexpr int NP = 16 * KPT;                 // padded headdim_qk
    static constexpr int PAIRS = NP / 2;
    static constexpr int PB = (PAIRS + 63) / 64;        // pairs per lane in the preparation
    static constexpr int TB = KPT >= 12 ? 16 : 32;      // tokens per block
    static constexpr int SEG = TB / kWaves;             // tokens per wave in the preparation
    static constexpr int TVP = (TB * kRows + kThreads - 1) / kThreads;   // V values per thread per block
    // gfx950 serves ds_read_b128 16 lanes at a time from 64 banks: for 8 and
    // 16 keys per lane, 16 bytes of padding per 256 bytes keep the 16 key
    // groups of a row on distinct banks.
    static constexpr bool PAD = KPT == 8 || KPT == 16 || KPT == 32;
    static constexpr int NPS = PAD ? NP + 4 * ((NP - 1) / 64) : NP;   // floats per token row of sQ / sK
    __host__ __device__ static constexpr int Pos(int i) { return PAD ? i + 4 * (i / 64) : i; }
    // dynamic LDS (bytes), doubles first
    static constexpr size_t kSeg = 0;                                          // double [kWaves][PAIRS]
    static constexpr size_t kCarry = kSeg + sizeof(double) * kWaves * PAIRS;   // double [2][PAIRS]
    static constexpr size_t kQ = kCarry + sizeof(double) * 2 * PAIRS;          // float [2][TB][NPS]
    static constexpr size_t kK = kQ + sizeof(float) * 2 * TB * NPS;            // float [2][TB][NPS]
    static constexpr size_t kV = kK + sizeof(float) * 2 * TB * NPS;            // float [2][TB][kRows]
    static constexpr size_t kScal = kV + sizeof(float) * 2 * TB * kRows;       // float [2][3][TB]
    static constexpr size_t kBytes = kScal + sizeof(float) * 2 * 3 * TB;
    static_assert(kQ % 16 == 0 && kK % 16 == 0 && kV % 16 == 0, "LDS regions must stay 16-byte aligned");
    static_assert(kBytes <= 160 * 1024, "LDS budget");
};

// k0_arg, nk_arg: the key block of this launch; first, last: whether it is
// the first / last block (KB only: otherwise every key, in one launch).
template <int KPT, bool KB>
__global__ __launch_bounds__(kThreads) void Mamba3FwdKernel(Mamba3SisoParams p, int k0_arg, int nk_arg, int first_arg,
                                                           int last_arg) {
    using L = M3Layout<KPT>;
    const int k0 = KB ? k0_arg : 0;                // first key of the block (even)
    const bool first = !KB || first_arg != 0, last = !KB || last_arg != 0;
    constexpr int PAIRS = L::PAIRS, PB = L::PB, TB = L::TB, SEG = L::SEG, NPS = L::NPS, TVP = L::TVP;

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    double *sSeg = reinterpret_cast<double *>(smem + L::kSeg);
    double *sCarry = reinterpret_cast<double *>(smem + L::kCarry);
    float *sQ = reinterpret_cast<float *>(smem + L::kQ);
    float *sK = reinterpret_cast<float *>(smem + L::kK);
    float *sV = reinterpret_cast<float *>(smem + L::kV);
    float *sScal = reinterpret_cast<float *>(smem + L::kScal);

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int N = p.n, P = p.p, A = p.a, H = p.nheads;   // N: the full headdim_qk (row strides)
    const int NK = KB ? nk_arg : N;                        // keys of this launch
    const int half_n = NK / 2;
    const int pa0 = k0 / 2;                                // first rotation pair of the block
    const int nrb = (P + kRows - 1) / kRows;
    // the nrb workgroups of one (b,h) prepare the same token vectors: keep them on one XCD
    const int wg = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int rb = wg % nrb;
    const int bh = wg / nrb;
    const int b = bh / H, h = bh % H;
    const int gq = h / (H / p.nheads_qk);
    const int r0 = rb * kRows;
    const float dval = (first && p.D) ? p.D[h] : 0.0f;
    // tokens of sequence b: [tok0, tok0 + T) of its token axis
    int T = p.seqlen;
    size_t tok0 = static_cast<size_t>(b) * T;    // in [B*T] for Q/K/V/Angles/Z
    size_t sbase = static_cast<size_t>(bh) * T;  // in [B*H*T] for ADT/DT/Trap
    if (p.cu_seqlens != nullptr) {
        const long long lo = min(max(p.cu_seqlens[b], 0LL), static_cast<long long>(p.seqlen));
        const long long hi = min(max(p.cu_seqlens[b + 1], lo), static_cast<long long>(p.seqlen));
        tok0 = static_cast<size_t>(lo);
        sbase = static_cast<size_t>(h) * p.seqlen + static_cast<size_t>(lo);
        T = static_cast<int>(hi - lo);
    }
    const float *dtr = p.DT + sbase;
    const float *trr = p.Trap + sbase;
    const float *adr = p.ADT + sbase;

    // ---- preparation state: lane handles pairs lane + 64*x, tokens w*SEG + s
    float2 qbias[PB], kbias[PB];
#pragma unroll
    for (int x = 0; x < PB; ++x) {
        const int pr = lane + 64 * x;
        const int pc = min(pr, half_n - 1);
        const float2 qb = *reinterpret_cast<const float2 *>(p.Q_bias + static_cast<size_t>(h) * N + k0 + 2 * pc);
        const float2 kb = *reinterpret_cast<const float2 *>(p.K_bias + static_cast<size_t>(h) * N + k0 + 2 * pc);
        const bool ok = pr < half_n;
        qbias[x] = ok ? qb : make_float2(0.0f, 0.0f);
        kbias[x] = ok ? kb : make_float2(0.0f, 0.0f);
    }
    // Per-token row bases and strides (elements); token t of this (b,h) is at base + t * stride.
    const size_t q_stride = static_cast<size_t>(p.nheads_qk) * N;
    const float *qbase = p.Q + (tok0 * p.nheads_qk + gq) * N + k0;
    const float *kbase = p.K + (tok0 * p.nheads_qk + gq) * N + k0;
    const size_t a_stride = static_cast<size_t>(H) * A;
    const float *abase = p.Angles + (tok0 * H + h) * A;
    const size_t v_stride = static_cast<size_t>(H) * P;
    const size_t vbase = (tok0 * H + h) * P;   // also the output / Z base

    // Raw prefetched values.  The loads use clamped addresses and nothing
    // selects on them until they are consumed after the recurrence: a select
    // next to the load lets the compiler sink the load into a branch and
    // wait for it on the spot, which would serialise the prefetch.
    float ang[PB][SEG], dts[SEG];
    float2 qv[PB][SEG], kv[PB][SEG];
    float vreg[TVP];
    float tdt = 0.0f, ttrap = 0.0f, tadt = 0.0f, tdt1 = 0.0f, ttrap1 = 0.0f;   // token scalars (lane < SEG)
    double pre[PB][SEG];

    // global -> registers for the block at t0
    auto load_prep = [&](int t0) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < SEG; ++s) {
            const int t = min(t0 + w * SEG + s, T - 1);
            dts[s] = dtr[t];
            const float *qr = qbase + static_cast<size_t>(t) * q_stride;
            const float *kr = kbase + static_cast<size_t>(t) * q_stride;
            const float *ar = abase + static_cast<size_t>(t) * a_stride;
#pragma unroll
            for (int x = 0; x < PB; ++x) {
                const int pr = lane + 64 * x;
                ang[x][s] = ar[min(pa0 + pr, A - 1)];
                const int pc = min(pr, half_n - 1);
                qv[x][s] = *reinterpret_cast<const float2 *>(qr + 2 * pc);
                kv[x][s] = *reinterpret_cast<const float2 *>(kr + 2 * pc);
            }
        }
        {
            const int t = min(t0 + w * SEG + min(lane, SEG - 1), T - 1);
            const int t1 = min(t + 1, T - 1);
            tdt = dtr[t];
            ttrap = trr[t];
            tadt = adr[t];
            tdt1 = dtr[t1];
            ttrap1 = trr[t1];
        }
#pragma unroll
        for (int k = 0; k < TVP; ++k) {
            const int i = tid + k * kThreads;
            const int t = min(t0 + i / kRows, T - 1);
            vreg[k] = p.V[vbase + static_cast<size_t>(t) * v_stride + min(r0 + i % kRows, P - 1)];
        }
    };

    // prep A: fp64 angle increments and their running sum over the wave's tokens
    auto prep_a = [&](int t0) __attribute__((always_inline)) {
        const int nt = min(TB, T - t0);
#pragma unroll
        for (int x = 0; x < PB; ++x) {
            const bool rot = pa0 + lane + 64 * x < A;
            double acc = 0.0;
#pragma unroll
            for (int s = 0; s < SEG; ++s) {
                const bool ok = rot && w * SEG + s < nt;
                const float a = ok ? ang[x][s] : 0.0f, d = ok ? dts[s] : 0.0f;
                acc += static_cast<double>(TanhF(a)) * static_cast<double>(d) * static_cast<double>(kPiF);
                pre[x][s] = acc;
            }
            const int pr = lane + 64 * x;
            if (pr < PAIRS) sSeg[w * PAIRS + pr] = acc;
        }
    };

    // prep B: wrapped angles, rotation, q.k and per-token scalars into buffer nb
    auto prep_b = [&](int t0, int nb, int cb) __attribute__((always_inline)) {
        const int nt = min(TB, T - t0);
        float qk[SEG];
#pragma unroll
        for (int s = 0; s < SEG; ++s) qk[s] = 0.0f;
#pragma unroll
        for (int x = 0; x < PB; ++x) {
            const int pr = lane + 64 * x;
            if (pr < PAIRS) {
                // earlier waves' sums: all reads issued at once, summed in wave order
                double carry = sCarry[cb * PAIRS + pr];
#pragma unroll
                for (int w2 = 0; w2 < kWaves - 1; ++w2) {
                    const double v = sSeg[w2 * PAIRS + pr];
                    carry = w2 < w ? carry + v : carry;
                }
                const bool rot = pa0 + pr < A;
                double th = 0.0;
#pragma unroll
                for (int s = 0; s < SEG; ++s) {
                    const int tt = w * SEG + s;
                    th = carry + pre[x][s];
                    // wrap_two_pi (reference :26-28); the reciprocal can move a wrap by one
                    // period only within an ulp of a multiple, where sin/cos agree
                    th -= kTwoPiF * floor(th * kInvTwoPiF);
                    float c = 1.0f, sn = 0.0f;
                    if (rot) {
                        const float rev = static_cast<float>(th * kRevPerRad);
                        sn = __builtin_amdgcn_sinf(rev);
                        c = __builtin_amdgcn_cosf(rev);
                    }
                    const bool okp = w * SEG + s < nt && pr < half_n;
                    const float2 q = okp ? make_float2(qv[x][s].x + qbias[x].x, qv[x][s].y + qbias[x].y)
                                         : make_float2(0.0f, 0.0f);
                    const float2 k = okp ? make_float2(kv[x][s].x + kbias[x].x, kv[x][s].y + kbias[x].y)
                                         : make_float2(0.0f, 0.0f);
                    qk[s] = fmaf(q.x, k.x, fmaf(q.y, k.y, qk[s]));   // unrotated q.k (reference :89-106)
                    const int o = (nb * TB + tt) * NPS + L::Pos(2 * pr);
                    *reinterpret_cast<float2 *>(&sQ[o]) = make_float2(q.x * c - q.y * sn, q.x * sn + q.y * c);
                    *reinterpret_cast<float2 *>(&sK[o]) = make_float2(k.x * c - k.y * sn, k.x * sn + k.y * c);
                }
                if (w == kWaves - 1) sCarry[(cb ^ 1) * PAIRS + pr] = rot ? th : 0.0;
            }
        }
        float myqk = 0.0f;
#pragma unroll
        for (int s = 0; s < SEG; ++s) {
            const float v = WaveSum64(qk[s]);
            myqk = lane == s ? v : myqk;
        }
        if (lane < SEG) {
            const int tt = w * SEG + lane;
            const int t = t0 + tt;
            const bool ok = tt < nt;
            const float gamma = tdt * FastSigmoid(ttrap);
            const float look = t + 1 < T ? tdt1 * (1.0f - FastSigmoid(ttrap1)) : 0.0f;
            float *sc = sScal + nb * 3 * TB;
            sc[tt] = ok ? __expf(tadt) : 1.0f;                // decay
            sc[TB + tt] = ok ? gamma + look : 0.0f;            // k scale
            sc[2 * TB + tt] = ok ? fmaf(myqk, gamma, dval) : 0.0f;   // D + qk * gamma
        }
#pragma unroll
        for (int k = 0; k < TVP; ++k) {
            const int i = tid + k * kThreads;
            if (i < TB * kRows) sV[nb * TB * kRows + i] = (i / kRows < nt && r0 + i % kRows < P) ? vreg[k] : 0.0f;
        }
    };

    // ---- recurrence
    const int kg = tid & 15, rg = tid >> 4;
    const int row = r0 + rg;
    const int kpos = L::Pos(kg * KPT);
    float S[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) S[j] = 0.0f;
    if (p.in_ssm != nullptr && row < P) {
        const float look0 = T > 0 ? dtr[0] * (1.0f - FastSigmoid(trr[0])) : 0.0f;   // stays pending when empty
        const float vl = p.in_v[static_cast<size_t>(bh) * P + row];
        const float *srow = p.in_ssm + (static_cast<size_t>(bh) * P + row) * N + k0;
        const float *krow = p.in_k + static_cast<size_t>(bh) * N + k0;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const int key = kg * KPT + j;
            if (key < NK) S[j] = fmaf(vl, krow[key] * look0, srow[key]);
        }
    }

    auto recur = [&](int t0, int buf) __attribute__((always_inline)) {
        const int nt = min(TB, T - t0);
        const float *qb = sQ + buf * TB * NPS + kpos;
        const float *kb = sK + buf * TB * NPS + kpos;
        const float *sc = sScal + buf * 3 * TB;
        const float *vr = sV + buf * TB * kRows + rg;
        float oreg[TB / 16];
#pragma unroll
        for (int u = 0; u < TB / 16; ++u) oreg[u] = 0.0f;
        // up to 16 keys per lane, token tt+1's q and k are read while token tt
        // computes; above that the second register set would spill, and each
        // token reads its own
        constexpr bool PREF = KPT <= 16;
        float cq[KPT], ck[KPT], nq[PREF ? KPT : 1], nk[PREF ? KPT : 1];
        float cdec, cks, cdiag, cv, ndec = 1.0f, nks = 0.0f, ndiag = 0.0f, nv = 0.0f;
        if constexpr (PREF) {
            LoadKeys<KPT>(qb, cq);
            LoadKeys<KPT>(kb, ck);
        }
        cdec = sc[0]; cks = sc[TB]; cdiag = sc[2 * TB]; cv = vr[0];
#pragma unroll
        for (int tt = 0; tt < TB; ++tt) {
            if constexpr (!PREF) LoadKeys<KPT>(qb + tt * NPS, cq);
            if (tt + 1 < TB) {
                if constexpr (PREF) {
                    LoadKeys<KPT>(qb + (tt + 1) * NPS, nq);
                    LoadKeys<KPT>(kb + (tt + 1) * NPS, nk);
                }
                ndec = sc[tt + 1]; nks = sc[TB + tt + 1]; ndiag = sc[2 * TB + tt + 1]; nv = vr[(tt + 1) * kRows];
            }
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int j = 0; j < KPT; j += 2) {
                S[j] *= cdec;                       // decay before the readout (reference :140-143)
                a0 = fmaf(cq[j], S[j], a0);
                if (j + 1 < KPT) {
                    S[j + 1] *= cdec;
                    a1 = fmaf(cq[j + 1], S[j + 1], a1);
                }
            }
            const float y = fmaf(cdiag, cv, RowSum16(a0 + a1));
            const float vk = cv * cks;
            if constexpr (!PREF) LoadKeys<KPT>(kb + tt * NPS, ck);   // after the readout: q and k not live together
#pragma unroll
            for (int j = 0; j < KPT; ++j) S[j] = fmaf(vk, ck[j], S[j]);   // S += V (x) k_rot (gamma + look)
            oreg[tt / 16] = kg == (tt & 15) ? y : oreg[tt / 16];
            if (tt + 1 < TB) {
                if constexpr (PREF) {
#pragma unroll
                    for (int j = 0; j < KPT; ++j) { cq[j] = nq[j]; ck[j] = nk[j]; }
                }
                cdec = ndec; cks = nks; cdiag = ndiag; cv = nv;
            }
        }
#pragma unroll
        for (int u = 0; u < TB / 16; ++u) {
            const int tt = u * 16 + kg;
            if (tt < nt && row < P) {
                const size_t idx = vbase + static_cast<size_t>(t0 + tt) * v_stride + row;
                float y = oreg[u];
                if (!first) y += p.out[idx];                 // the earlier key blocks' part
                if (last && p.Z) {
                    const float z = p.Z[idx];
                    y *= z * FastSigmoid(z);                 // silu gate (reference :155-158)
                }
                p.out[idx] = y;
            }
        }
    };

    if (tid < PAIRS)
        sCarry[tid] = (p.in_angle != nullptr && pa0 + tid < A) ? static_cast<double>(p.in_angle[static_cast<size_t>(bh) * A + pa0 + tid]) : 0.0;
    const int nblk = (T + TB - 1) / TB;
    if (T > 0) {   // workgroup-uniform: an empty sequence passes its states through
        load_prep(0);
        prep_a(0);
        __syncthreads();
        prep_b(0, 0, 0);
        __syncthreads();
        for (int j = 0; j < nblk; ++j) {
            const int buf = j & 1;
            const bool next = j + 1 < nblk;
            if (next) load_prep((j + 1) * TB);
            recur(j * TB, buf);
            if (next) prep_a((j + 1) * TB);
            __syncthreads();
            if (next) prep_b((j + 1) * TB, buf ^ 1, (j + 1) & 1);
            __syncthreads();
        }
    } else {
        __syncthreads();   // the initial angle carry, read back below
    }
    if (p.f_ssm != nullptr) {
        // the last block's buffers are intact: sK holds its rotated k, the
        // carry of parity nblk % 2 the wrapped angle after its last token
        if (row < P) {
            float *srow = p.f_ssm + (static_cast<size_t>(bh) * P + row) * N + k0;
#pragma unroll
            for (int j = 0; j < KPT; ++j)
                if (kg * KPT + j < NK) srow[kg * KPT + j] = S[j];
        }
        if (tid < kRows && r0 + tid < P) {
            const size_t o = static_cast<size_t>(bh) * P + r0 + tid;
            p.f_v[o] = T > 0 ? p.V[vbase + static_cast<size_t>(T - 1) * v_stride + r0 + tid]
                             : (p.in_v != nullptr ? p.in_v[o] : 0.0f);
        }
        if (rb == 0) {
            const int tl = T > 0 ? (T - 1) - (nblk - 1) * TB : 0;
            const float *krow = sK + (((nblk - 1) & 1) * TB + tl) * NPS;
            for (int i = tid; i < NK; i += kThreads) {
                const size_t o = static_cast<size_t>(bh) * N + k0 + i;
                p.f_k[o] = T > 0 ? krow[L::Pos(i)] : (p.in_k != nullptr ? p.in_k[o] : 0.0f);
            }
            for (int i = tid; i < half_n && pa0 + i < A; i += kThreads)
                p.f_angle[static_cast<size_t>(bh) * A + pa0 + i] = static_cast<float>(sCarry[(nblk & 1) * PAIRS + i]);
        }
    }
}

template <int KPT, bool KB = false>
void LaunchKPT(const Mamba3SisoParams &p, hipStream_t stream, int k0 = 0, int nk = 0, bool first = true,
               bool last = true) {
    using L = M3Layout<KPT>;
    const long long blocks = static_cast<long long>(p.batch) * p.nheads * ((p.p + kRows - 1) / kRows);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "Mamba3SisoFn launch exceeds the grid limit");
    EnsureDynamicLds(reinterpret_cast<const void *>(&Mamba3FwdKernel<KPT, KB>), static_cast<int>(L::kBytes));
    if constexpr (KB) XM_NOTE_LAUNCH("Mamba3FwdKernel", {}, KPT, 1);
    else XM_NOTE_LAUNCH("Mamba3FwdKernel", {}, KPT);
    hipLaunchKernelGGL((Mamba3FwdKernel<KPT, KB>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), L::kBytes, stream, p,
                       k0, nk, first ? 1 : 0, last ? 1 : 0);
}

constexpr int kKeyBlock = 16 * 32;   // keys per launch above 512 (32 per lane of a 16-lane row)

}  // namespace

void LaunchMamba3Siso(const Mamba3SisoParams &p, void *stream_v) {
    // packed: token rows outside every sequence are zeros, not left unwritten
    if (p.cu_seqlens != nullptr)
        LaunchPackedGaps(p.out, static_cast<size_t>(p.nheads) * p.p, p.cu_seqlens, p.batch, p.seqlen, stream_v);
    if (LaunchMamba3SisoChunked(p, stream_v)) return;
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    const int kpt = (p.n + 15) / 16;
    if (kpt <= 4) LaunchKPT<4>(p, stream);
    else if (kpt <= 8) LaunchKPT<8>(p, stream);
    else if (kpt <= 12) LaunchKPT<12>(p, stream);
    else if (kpt <= 16) LaunchKPT<16>(p, stream);
    else if (kpt <= 24) LaunchKPT<24>(p, stream);
    else if (kpt <= 32) LaunchKPT<32>(p, stream);
    else
        for (int k0 = 0; k0 < p.n; k0 += kKeyBlock)   // stream order: each launch adds to the earlier ones' y
            LaunchKPT<32, true>(p, stream, k0, std::min(kKeyBlock, p.n - k0), k0 == 0, k0 + kKeyBlock >= p.n);
    XM_LAUNCH_CHECK("Mamba3SisoFn");
}

}  // namespace xm
