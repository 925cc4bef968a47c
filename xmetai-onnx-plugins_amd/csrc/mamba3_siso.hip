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
// One fused kernel; a workgroup owns one (b,h) and a block of 16*RPT state
// rows, and walks the sequence in blocks of kTB tokens:
//   A) angle scan: tanh(Angles)*DT*pi for every (token, pair) in parallel,
//      then one lane per pair accumulates in fp64 and wraps, so the angle
//      state carries no fp32 round-off from step to step;
//   B) one wave per token: bias add, q.k (wave reduction), rotation,
//      trapezoid coefficients, decay and diagonal term -> LDS;
//   C) recurrence: lane (row group, key group) holds RPT rows x KPT keys of
//      S in VGPRs; the readout over keys is a 4-step DPP row sum;
//   D) y = readout + diag*V (* silu(Z)), stored with coalesced rows.
// Pairs >= A are not rotated (reference :109).
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "xm_hip.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr int kThreads = 256;
constexpr int kTB = 16;                 // tokens per block
constexpr float kPiF = 3.14159265358979323846f;      // reference kPi (mamba3_siso_fwd.cu:15)
constexpr double kTwoPiD = 2.0 * static_cast<double>(kPiF);  // reference kTwoPi = 2 * kPi

__device__ __forceinline__ float Sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

template <int KPT, int RPT>
__global__ __launch_bounds__(kThreads) void Mamba3FwdKernel(Mamba3SisoParams p) {
    constexpr int NP = 16 * KPT;        // padded headdim_qk
    constexpr int PAIRS = NP / 2;
    constexpr int RB = 16 * RPT;        // state rows per workgroup

    __shared__ __attribute__((aligned(16))) float sQ[kTB * NP];   // rotated q
    __shared__ __attribute__((aligned(16))) float sK[kTB * NP];   // rotated k * (gamma + look)
    __shared__ float sV[kTB * RB];
    __shared__ float sZ[kTB * RB];
    __shared__ float sY[kTB * RB];
    __shared__ float sDecay[kTB], sDiag[kTB];
    __shared__ float sTh[kTB * PAIRS];      // wrapped angle per (token, pair)
    __shared__ double sDelta[kTB * PAIRS];  // angle increments
    __shared__ double sCarry[PAIRS];        // angle state at the end of the previous block

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int T = p.seqlen, N = p.n, P = p.p, A = p.a;
    const int nrb = (P + RB - 1) / RB;
    // the nrb workgroups of one (b,h) read the same token vectors: keep them on one XCD
    const int wg = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int rb = wg % nrb;
    const int bh = wg / nrb;
    const int b = bh / p.nheads, h = bh % p.nheads;
    const int gq = h / (p.nheads / p.nheads_qk);
    const int r0 = rb * RB;
    const bool has_z = p.Z != nullptr;
    const float dval = p.D ? p.D[h] : 0.0f;

    const float *dtr = p.DT + static_cast<size_t>(bh) * T;
    const float *trr = p.Trap + static_cast<size_t>(bh) * T;
    const float *adr = p.ADT + static_cast<size_t>(bh) * T;

    // Recurrence lane layout: kg = key group (16 lanes of a DPP row), rg = row group.
    const int kg = tid & 15, rg = tid >> 4;
    float S[RPT][KPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int j = 0; j < KPT; ++j) S[i][j] = 0.0f;
    for (int i = tid; i < PAIRS; i += kThreads) sCarry[i] = 0.0;

    for (int t0 = 0; t0 < T; t0 += kTB) {
        const int nt = min(kTB, T - t0);

        // ---- A1: angle increments tanh(angle) * dt * pi (fp32 tanh, fp64 products)
        for (int i = tid; i < kTB * PAIRS; i += kThreads) {
            const int tt = i / PAIRS, pr = i % PAIRS;
            double dlt = 0.0;
            if (tt < nt && pr < A) {
                const int t = t0 + tt;
                const float ang = p.Angles[((static_cast<size_t>(b) * T + t) * p.nheads + h) * A + pr];
                dlt = static_cast<double>(tanhf(ang)) * static_cast<double>(dtr[t]) * static_cast<double>(kPiF);
            }
            sDelta[i] = dlt;
        }
        // V and Z rows of this block (coalesced: RB contiguous floats per token).
        for (int i = tid; i < kTB * RB; i += kThreads) {
            const int tt = i / RB, r = r0 + i % RB;
            float vv = 0.0f, zz = 0.0f;
            if (tt < nt && r < P) {
                const size_t idx = ((static_cast<size_t>(b) * T + t0 + tt) * p.nheads + h) * P + r;
                vv = p.V[idx];
                if (has_z) zz = p.Z[idx];
            }
            sV[i] = vv;
            sZ[i] = zz;
        }
        __syncthreads();

        // ---- A2: sequential wrap per pair, in fp64 (reference :82-86, :26-28)
        for (int pr = tid; pr < A; pr += kThreads) {
            double th = sCarry[pr];
            for (int tt = 0; tt < nt; ++tt) {
                th += sDelta[tt * PAIRS + pr];
                th -= kTwoPiD * floor(th * (1.0 / kTwoPiD));
                sTh[tt * PAIRS + pr] = static_cast<float>(th);
            }
            sCarry[pr] = th;
        }
        __syncthreads();

        // ---- B: per-token vectors, one wave per token
        for (int tt = w; tt < nt; tt += kThreads / 64) {
            const int t = t0 + tt;
            const size_t qrow = ((static_cast<size_t>(b) * T + t) * p.nheads_qk + gq) * N;
            float qk = 0.0f;
            float2 qv[(PAIRS + 63) / 64], kv[(PAIRS + 63) / 64];
#pragma unroll
            for (int x = 0; x < (PAIRS + 63) / 64; ++x) {
                const int pr = lane + 64 * x;
                float2 qq = make_float2(0.0f, 0.0f), kk = make_float2(0.0f, 0.0f);
                if (pr < N / 2) {
                    const float2 q2 = *reinterpret_cast<const float2 *>(p.Q + qrow + 2 * pr);
                    const float2 k2 = *reinterpret_cast<const float2 *>(p.K + qrow + 2 * pr);
                    const float2 qb = *reinterpret_cast<const float2 *>(p.Q_bias + static_cast<size_t>(h) * N + 2 * pr);
                    const float2 kb = *reinterpret_cast<const float2 *>(p.K_bias + static_cast<size_t>(h) * N + 2 * pr);
                    qq = make_float2(q2.x + qb.x, q2.y + qb.y);
                    kk = make_float2(k2.x + kb.x, k2.y + kb.y);
                    qk = fmaf(qq.x, kk.x, qk);
                    qk = fmaf(qq.y, kk.y, qk);
                }
                qv[x] = qq;
                kv[x] = kk;
            }
            qk = WaveSum64(qk);   // unrotated q.k (reference :89-106)
            const float dt = dtr[t];
            const float gamma = dt * Sigmoid(trr[t]);
            float look = 0.0f;
            if (t + 1 < T) look = dtr[t + 1] * (1.0f - Sigmoid(trr[t + 1]));
            const float kscale = gamma + look;
#pragma unroll
            for (int x = 0; x < (PAIRS + 63) / 64; ++x) {
                const int pr = lane + 64 * x;
                if (pr < PAIRS) {
                    float c = 1.0f, s = 0.0f;
                    if (pr < A) sincosf(sTh[tt * PAIRS + pr], &s, &c);
                    const float2 qq = qv[x], kk = kv[x];
                    sQ[tt * NP + 2 * pr] = qq.x * c - qq.y * s;
                    sQ[tt * NP + 2 * pr + 1] = qq.x * s + qq.y * c;
                    sK[tt * NP + 2 * pr] = (kk.x * c - kk.y * s) * kscale;
                    sK[tt * NP + 2 * pr + 1] = (kk.x * s + kk.y * c) * kscale;
                }
            }
            if (lane == 0) {
                sDecay[tt] = expf(adr[t]);
                sDiag[tt] = dval + qk * gamma;
            }
        }
        __syncthreads();

        // ---- C: recurrence over the block
        for (int tt = 0; tt < nt; ++tt) {
            const float dec = sDecay[tt];
            float q[KPT], k[KPT];
#pragma unroll
            for (int j = 0; j < KPT; j += 4) {
                const float4 a = *reinterpret_cast<const float4 *>(&sQ[tt * NP + kg * KPT + j]);
                const float4 c = *reinterpret_cast<const float4 *>(&sK[tt * NP + kg * KPT + j]);
                q[j] = a.x; q[j + 1] = a.y; q[j + 2] = a.z; q[j + 3] = a.w;
                k[j] = c.x; k[j + 1] = c.y; k[j + 2] = c.z; k[j + 3] = c.w;
            }
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                const int rl = rg * RPT + i;
                const float vv = sV[tt * RB + rl];
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < KPT; ++j) {
                    S[i][j] *= dec;
                    acc = fmaf(q[j], S[i][j], acc);
                }
                acc = RowSum16(acc);
#pragma unroll
                for (int j = 0; j < KPT; ++j) S[i][j] = fmaf(vv, k[j], S[i][j]);
                if (kg == 0) sY[tt * RB + rl] = acc;
            }
        }
        __syncthreads();

        // ---- D: y = readout + diag * V, optional silu(Z) gate; coalesced store
        for (int i = tid; i < nt * RB; i += kThreads) {
            const int tt = i / RB, r = r0 + i % RB;
            if (r < P) {
                float y = sY[i] + sDiag[tt] * sV[i];
                if (has_z) {
                    const float z = sZ[i];
                    y *= z * Sigmoid(z);
                }
                p.out[((static_cast<size_t>(b) * T + t0 + tt) * p.nheads + h) * P + r] = y;
            }
        }
        // Next block's phase A writes sDelta/sV/sZ (last read before the
        // barrier above) and sTh/sQ/sK/sY only after further barriers.
        __syncthreads();
    }
}

template <int KPT>
void LaunchKPT(const Mamba3SisoParams &p, int rpt, hipStream_t stream) {
    if (KPT >= 12 && rpt == 4) rpt = 2;
    const int rb = 16 * rpt;
    const long long blocks = static_cast<long long>(p.batch) * p.nheads * ((p.p + rb - 1) / rb);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "Mamba3SisoFn launch exceeds the grid limit");
    const dim3 grid(static_cast<unsigned>(blocks));
    if (rpt == 1) {
        hipLaunchKernelGGL((Mamba3FwdKernel<KPT, 1>), grid, dim3(kThreads), 0, stream, p);
    } else if (rpt == 2 || KPT >= 12) {
        // 4 rows per lane would exceed 64 KiB of LDS for headdim_qk > 128
        hipLaunchKernelGGL((Mamba3FwdKernel<KPT, 2>), grid, dim3(kThreads), 0, stream, p);
    } else {
        if constexpr (KPT < 12) hipLaunchKernelGGL((Mamba3FwdKernel<KPT, 4>), grid, dim3(kThreads), 0, stream, p);
    }
}

// Rows per lane (16 rows per workgroup per row per lane).  XM_M3_RPT (1, 2
// or 4) overrides, for tuning.
int RowsPerLane(const Mamba3SisoParams &p) {
    const char *env = std::getenv("XM_M3_RPT");
    const int forced = env ? std::atoi(env) : 0;
    if (forced == 1 || forced == 2 || forced == 4) return forced;
    (void)p;
    return 1;   // measured fastest at 4 x 4096 x 32 heads, P = 64, N = 128
}

}  // namespace

void LaunchMamba3Siso(const Mamba3SisoParams &p, void *stream_v) {
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    const int rpt = RowsPerLane(p);
    const int kpt = (p.n + 15) / 16;
    if (kpt <= 4) LaunchKPT<4>(p, rpt, stream);
    else if (kpt <= 8) LaunchKPT<8>(p, rpt, stream);
    else if (kpt <= 12) LaunchKPT<12>(p, rpt, stream);
    else LaunchKPT<16>(p, rpt, stream);
    XM_LAUNCH_CHECK("Mamba3SisoFn");
}

}  // namespace xm
