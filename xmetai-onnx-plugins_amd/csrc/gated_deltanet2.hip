// GatedDeltaNet2Fn forward for gfx950 (CDNA4, wave64).
//
// Math (reference gated_deltanet2_fwd.cu:39-140, identical in :142-233):
// per (b,h) a dk x dv state S; per token
//     qhat = q*scale*rsqrt(|q|^2+1e-6), khat = k*rsqrt(|k|^2+1e-6)  (when L2 norm is on)
//     S[i,:] *= exp(g_i);  e_j = sum_i beta_i khat_i S[i,j];  u_j = w_j v_j - e_j
//     S[i,j] += khat_i u_j; o_j = sum_i qhat_i S[i,j]
// Every value column j evolves independently given the per-token vectors.
//
// Evaluation order on the device.  With d = exp(g) and S the state before
// the token, both sums the token needs read the same S:
//     e_j = sum_i (beta_i khat_i d_i) S[i,j]       r_j = sum_i (qhat_i d_i) S[i,j]
//     u_j = w_j v_j - e_j                          o_j = r_j + (qhat . khat) u_j
//     S[i,j] <- fma(khat_i, u_j, S[i,j] * d_i)     (the reference's decay-then-update)
// so one cross-lane reduction phase (of two values) per token sits on the
// recurrence's critical path instead of two, and the readout leaves it.  The
// state itself is updated with the reference's operations; e and o differ from
// the reference only in the association of their products.
//
// Kernels:
//  * Gdn2FusedKernel (dk <= 512): one launch for the whole sequence, no
//    scratch.  A workgroup of NW waves owns 4*NW/R value columns of one
//    (b,h); a column spans R = 1, 2 or 4 rows of 16 lanes that split its keys
//    (KT each), so the reduction over keys is a 4-step DPP row sum plus one
//    or two lane swaps.  The state lives in VGPRs.  Tokens run in blocks of NW: wave w prepares token w of the next
//    block (L2 norms, exp(g), the four vectors, qhat.khat, w*v) into
//    double-buffered LDS while the current block's recurrence runs.
//  * Gdn2PrepKernel + Gdn2RecurLdsKernel (dk > 512): the preparation writes
//    khat, beta*khat*d, qhat*d, d and qhat.khat for a chunk of <= 1024 tokens
//    to scratch; the recurrence keeps the [dk_pad x 16 columns] state tile in
//    LDS and carries the fp32 state across chunks through scratch
//    (reference :101-102, :133-139).  Above 2048 keys the tile (128 KiB at
//    2048) no longer fits in LDS: the same recurrence then keeps it in a
//    scratch region of its own (Gdn2RecurLdsKernel<true>), in the tile's
//    lane order, so a wave's state accesses stay 256-byte contiguous; the
//    region also carries the state across chunks.  Its preparation loops over
//    the keys (Gdn2PrepLoopKernel).  This is the reference's generic kernel's
//    arrangement (state in global memory, gated_deltanet2_fwd.cu:142-233),
//    with no key limit.
//  * The tokens per preparation chunk (<= 1024) follow from the scratch bytes
//    available: a caller with a fixed scratch budget gets shorter chunks.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "xm_hip.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr int kThreads = 256;
constexpr int kChunkTokens = 1024;   // reference kGatedDeltaNet2PrepareTokens (gated_deltanet2.h:11)
constexpr int kFusedKeyLimit = 512;  // register-state kernel: up to 4 rows x 16 lanes x 8 keys per column
                                     // (the reference's register path stops at 256, gated_deltanet2.h:10)
constexpr int kMaxLdsKeys = 2048;    // LDS-state tile: dk_pad * 16 columns * 4 B <= 128 KiB; above, scratch
constexpr float kL2Eps = 1.0e-6f;    // reference kL2NormEps (gated_deltanet2_fwd.cu:14)

// Prepared row of one (b,h,t): [khat | beta*khat*d | qhat*d | d], kp floats
// each; qhat.khat of the row goes to a separate per-(b,h,t) array (p.prep_qk).
__host__ __device__ constexpr int PrepRow(int kp) { return 4 * kp; }

// ---------------------------------------------------------------------------
// Preparation
// ---------------------------------------------------------------------------
template <int KPL>
__global__ __launch_bounds__(kThreads) void Gdn2PrepKernel(GatedDeltaNet2Params p, int t0, int tc) {
    const int lane = threadIdx.x & 63;
    const long long row = static_cast<long long>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    const long long rows = static_cast<long long>(p.batch) * p.nheads * tc;
    if (row >= rows) return;  // uniform per wave
    const int tl = static_cast<int>(row % tc);
    const int bh = static_cast<int>(row / tc);
    const int b = bh / p.nheads, h = bh % p.nheads;
    const int t = t0 + tl;
    const int dk = p.dk, kp = p.dk_pad;
    const size_t src = ((static_cast<size_t>(b) * p.seqlen + t) * p.nheads + h) * static_cast<size_t>(dk);
    float q[KPL], k[KPL];
    float qs = 0.0f, ks = 0.0f;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
        const int kd = lane + 64 * j;
        q[j] = kd < dk ? p.q[src + kd] : 0.0f;
        k[j] = kd < dk ? p.k[src + kd] : 0.0f;
        qs = fmaf(q[j], q[j], qs);
        ks = fmaf(k[j], k[j], ks);
    }
    float q_mul = p.scale, k_mul = 1.0f;
    if (p.l2norm) {
        // reference :58-62: q_mul = scale * rsqrt(sum + eps); k_mul = rsqrt(sum + eps)
        q_mul *= rsqrtf(WaveSum64(qs) + kL2Eps);
        k_mul = rsqrtf(WaveSum64(ks) + kL2Eps);
    }
    float *dst = p.prepared + (static_cast<size_t>(bh) * p.chunk_cap + tl) * static_cast<size_t>(PrepRow(kp));
    float qk = 0.0f;
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
        const int kd = lane + 64 * j;
        if (kd < kp) {
            const bool ok = kd < dk;
            const float kn = ok ? k[j] * k_mul : 0.0f;                 // khat
            const float qn = ok ? q[j] * q_mul : 0.0f;                 // qhat
            const float d = ok ? expf(p.g[src + kd]) : 0.0f;           // exp(g)
            const float bk = ok ? p.beta[src + kd] * kn : 0.0f;        // beta * khat
            dst[kd] = kn;
            dst[kp + kd] = bk * d;
            dst[2 * kp + kd] = qn * d;
            dst[3 * kp + kd] = d;
            qk = fmaf(qn, kn, qk);
        }
    }
    qk = WaveSum64(qk);
    if (lane == 0) p.prep_qk[static_cast<size_t>(bh) * p.chunk_cap + tl] = qk;
}

// The same preparation for any dk (dk_pad > 2048): one wave per row, the sums
// of squares in a first pass over the keys and the four vectors in a second
// (the row is re-read from cache).
__global__ __launch_bounds__(kThreads) void Gdn2PrepLoopKernel(GatedDeltaNet2Params p, int t0, int tc) {
    const int lane = threadIdx.x & 63;
    const long long row = static_cast<long long>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    const long long rows = static_cast<long long>(p.batch) * p.nheads * tc;
    if (row >= rows) return;  // uniform per wave
    const int tl = static_cast<int>(row % tc);
    const int bh = static_cast<int>(row / tc);
    const int b = bh / p.nheads, h = bh % p.nheads;
    const int t = t0 + tl;
    const int dk = p.dk, kp = p.dk_pad;
    const size_t src = ((static_cast<size_t>(b) * p.seqlen + t) * p.nheads + h) * static_cast<size_t>(dk);
    float qs = 0.0f, ks = 0.0f;
    for (int kd = lane; kd < dk; kd += 64) {
        const float q = p.q[src + kd], k = p.k[src + kd];
        qs = fmaf(q, q, qs);
        ks = fmaf(k, k, ks);
    }
    float q_mul = p.scale, k_mul = 1.0f;
    if (p.l2norm) {
        // reference :58-62: q_mul = scale * rsqrt(sum + eps); k_mul = rsqrt(sum + eps)
        q_mul *= rsqrtf(WaveSum64(qs) + kL2Eps);
        k_mul = rsqrtf(WaveSum64(ks) + kL2Eps);
    }
    float *dst = p.prepared + (static_cast<size_t>(bh) * p.chunk_cap + tl) * static_cast<size_t>(PrepRow(kp));
    float qk = 0.0f;
    for (int kd = lane; kd < kp; kd += 64) {
        const bool ok = kd < dk;
        const float kn = ok ? p.k[src + kd] * k_mul : 0.0f;           // khat
        const float qn = ok ? p.q[src + kd] * q_mul : 0.0f;           // qhat
        const float d = ok ? expf(p.g[src + kd]) : 0.0f;              // exp(g)
        const float bk = ok ? p.beta[src + kd] * kn : 0.0f;           // beta * khat
        dst[kd] = kn;
        dst[kp + kd] = bk * d;
        dst[2 * kp + kd] = qn * d;
        dst[3 * kp + kd] = d;
        qk = fmaf(qn, kn, qk);
    }
    qk = WaveSum64(qk);
    if (lane == 0) p.prep_qk[static_cast<size_t>(bh) * p.chunk_cap + tl] = qk;
}

// ---------------------------------------------------------------------------
// Fused register-state kernel (dk <= 512): preparation + recurrence
// ---------------------------------------------------------------------------
// LDS layout of one staged token for KT keys per lane and R rows of 16 lanes
// per value column: each of the 4 vectors occupies KPS floats.  gfx950 serves
// a ds_read_b128 16 lanes (one row) at a time from 64 four-byte banks, so the
// 16 key groups of a row are conflict-free when their 16-byte chunks land on
// distinct (address/16) mod 16 slots.  KT = 4 (contiguous) and KT = 12
// (stride 3 chunks) already do, as do the 8-byte reads of KT = 2 and 6; KT =
// 8 and 16 would alias 2- and 4-way, so key i is stored at i + 4*(i/64) (16
// bytes of padding per 256 bytes) for them.
template <int KT, int R>
struct Swz {
    static constexpr int KP = 16 * R * KT;
    static constexpr bool PAD = KT == 8 || KT == 16;
    static constexpr int KPS = PAD ? KP + 4 * ((KP - 1) / 64) : KP;
    static constexpr int RS = 4 * KPS;
    __device__ static constexpr int Pos(int i) { return PAD ? i + 4 * (i / 64) : i; }
};

// NW waves per workgroup; a value column spans R rows of 16 lanes (R = 1,
// 2 or 4, all in one wave), so a workgroup has 4*NW/R columns.  Blocks of
// TB = NW * TPW tokens: wave w prepares tokens w*TPW .. w*TPW + TPW - 1.  The
// 4-wave workgroups (small problems) take two tokens per wave where the
// double-buffered staging fits in LDS: measured 4% faster there (longer blocks
// hide the next block's HBM prefetch), 1% slower with 8 waves.
template <int KT, int NW, int R>
struct FusedLayout {
    static constexpr int KP = Swz<KT, R>::KP;
    static constexpr int RS = Swz<KT, R>::RS;              // floats per staged token
    static constexpr int TPW = NW == 4 && 2 * 2 * NW * RS * sizeof(float) <= 150 * 1024 ? 2 : 1;
    static constexpr int TB = NW * TPW;                    // tokens per block (<= 16)
    static constexpr int THREADS = 64 * NW;
    static constexpr int COLS = 4 * NW / R;                // value columns per workgroup
    static constexpr int KPL = (KP + 63) / 64;             // keys per lane in the preparation
    static constexpr int WVPT = (TB * COLS + THREADS - 1) / THREADS;
    static constexpr size_t kVec = 0;                                   // float [2][TB][RS]
    static constexpr size_t kWV = kVec + sizeof(float) * 2 * TB * RS;   // float [2][TB][COLS]
    static constexpr size_t kQK = kWV + sizeof(float) * 2 * TB * COLS;  // float [2][TB]
    static constexpr size_t kBytes = kQK + sizeof(float) * 2 * TB;
    static_assert(kBytes <= 160 * 1024, "LDS budget");
};

// Sum over the R*16 lanes of one value column (rows 2c.. or all 4 rows), in
// every lane of the column: the row sum, then the gfx950 lane swaps
// (permlane16_swap pairs rows 0-1 and 2-3, permlane32_swap the two halves).
template <int R>
__device__ __forceinline__ float ColumnSum(float x) {
    x = RowSum16(x);
    if constexpr (R >= 2) {
        const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    }
    if constexpr (R == 4) {
        const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = __uint_as_float(s[0]) + __uint_as_float(s[1]);
    }
    return x;
}

template <int KT, int NW, int R>
__global__ __launch_bounds__(64 * NW) void Gdn2FusedKernel(GatedDeltaNet2Params p) {
    using L = FusedLayout<KT, NW, R>;
    using S_ = Swz<KT, R>;
    constexpr int KP = L::KP, KPS = S_::KPS, RS = L::RS, TB = L::TB, COLS = L::COLS;
    constexpr int KPL = L::KPL, THREADS = L::THREADS, WVPT = L::WVPT, TPW = L::TPW;
    static_assert(TB <= 16, "lane kg keeps the output of token kg of a block");

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    float *sVec = reinterpret_cast<float *>(smem + L::kVec);
    float *sWV = reinterpret_cast<float *>(smem + L::kWV);
    float *sQK = reinterpret_cast<float *>(smem + L::kQK);

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int kg = lane & 15;
    const int grow = w * 4 + (lane >> 4);         // 16-lane row within the workgroup
    const int cl = grow / R;                      // column within the workgroup
    const int rho = grow % R;                     // row within the column
    const int kb = (rho * 16 + kg) * KT;          // first of this lane's KT keys
    const int H = p.nheads, dk = p.dk, dv = p.dv;
    const int nvb = (dv + COLS - 1) / COLS;
    // the nvb workgroups of one (b,h) prepare the same token vectors: keep them on one XCD
    const int wg = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int vb = wg % nvb;
    const int bh = wg / nvb;
    const int b = bh / H, h = bh % H;
    // tokens of sequence b: [tok0, tok0 + T) of the token axis (packed
    // sequences: offsets clamped into [0, seqlen], an inverted range is empty)
    int T = p.seqlen;
    size_t tok0 = static_cast<size_t>(b) * T;
    if (p.cu_seqlens != nullptr) {
        const long long lo = min(max(p.cu_seqlens[b], 0LL), static_cast<long long>(p.seqlen));
        const long long hi = min(max(p.cu_seqlens[b + 1], lo), static_cast<long long>(p.seqlen));
        tok0 = static_cast<size_t>(lo);
        T = static_cast<int>(hi - lo);
    }
    const int v0 = vb * COLS;
    const int col = v0 + cl;                      // this lane's value column

    float S[KT];
    const size_t sbase = static_cast<size_t>(bh) * dk * dv;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const int kd = kb + j;
        S[j] = (p.initial_state && kd < dk && col < dv) ? p.initial_state[sbase + static_cast<size_t>(kd) * dv + col] : 0.0f;
    }

    // token t of (b,h): q/k/g/beta row at kbase + t*kstride, v/w/out row at vbase + t*vstride
    const size_t kstride = static_cast<size_t>(H) * dk, vstride = static_cast<size_t>(H) * dv;
    const size_t kbase = (tok0 * H + h) * dk;
    const size_t vbase = (tok0 * H + h) * dv;
    auto key = [&](int x) __attribute__((always_inline)) { return lane * KPL + x; };

    // Raw rows of the next block, loaded before the current block's recurrence
    // and consumed after it.  Clamped addresses, no selects here: a select
    // next to a load lets the compiler sink the load and wait on the spot.
    float rq[TPW][KPL], rk[TPW][KPL], rgd[TPW][KPL], rbt[TPW][KPL], rw[WVPT], rv[WVPT];
    auto load_block = [&](int t0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const size_t base = kbase + static_cast<size_t>(min(t0 + w * TPW + i, T - 1)) * kstride;
#pragma unroll
            for (int x = 0; x < KPL; ++x) {
                const int kc = min(key(x), dk - 1);
                rq[i][x] = p.q[base + kc];
                rk[i][x] = p.k[base + kc];
                rgd[i][x] = p.g[base + kc];
                rbt[i][x] = p.beta[base + kc];
            }
        }
#pragma unroll
        for (int k = 0; k < WVPT; ++k) {
            const int i = tid + k * THREADS;
            const int t = min(t0 + min(i / COLS, TB - 1), T - 1);
            const size_t idx = vbase + static_cast<size_t>(t) * vstride + min(v0 + i % COLS, dv - 1);
            rw[k] = p.w[idx];
            rv[k] = p.v[idx];
        }
    };

    // Preparation of one block into LDS buffer `buf` (reference :39-76):
    // qhat = q*scale*rsqrt(|q|^2+eps), khat = k*rsqrt(|k|^2+eps), d = exp(g), and
    // the staged vectors [khat | beta*khat*d | qhat*d | d] plus qhat.khat and w*v.
    // Tokens past the end are identity tokens (zero vectors, d = 1, w*v = 0):
    // they leave a finite state exactly unchanged.
    auto prep_block = [&](int t0, int buf) __attribute__((always_inline)) {
        const int nt = min(TB, T - t0);
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int tt = w * TPW + i;
            const bool live = tt < nt;                // wave-uniform
            float q[KPL], k[KPL];
            float qs = 0.0f, ks = 0.0f;
#pragma unroll
            for (int x = 0; x < KPL; ++x) {
                const bool ok = live && key(x) < dk;
                q[x] = ok ? rq[i][x] : 0.0f;
                k[x] = ok ? rk[i][x] : 0.0f;
                qs = fmaf(q[x], q[x], qs);
                ks = fmaf(k[x], k[x], ks);
            }
            float q_mul = p.scale, k_mul = 1.0f;
            if (p.l2norm) {
                // reference :58-62: q_mul = scale * rsqrt(sum + eps); k_mul = rsqrt(sum + eps)
                q_mul *= rsqrtf(WaveSum64(qs) + kL2Eps);
                k_mul = rsqrtf(WaveSum64(ks) + kL2Eps);
            }
            float *vt = sVec + (buf * TB + tt) * RS;
            float qk = 0.0f;
#pragma unroll
            for (int x = 0; x < KPL; ++x) {
                const int kd = key(x);
                if (kd < KP) {
                    const bool ok = live && kd < dk;
                    const float kn = k[x] * k_mul;                         // khat
                    const float qn = q[x] * q_mul;                         // qhat
                    // exp(g), hardware exp2 (the reference is built with fast math)
                    const float d = ok ? __expf(rgd[i][x]) : (live ? 0.0f : 1.0f);
                    const float bk = ok ? rbt[i][x] * kn : 0.0f;           // beta * khat
                    const int pos = S_::Pos(kd);
                    vt[pos] = kn;
                    vt[KPS + pos] = bk * d;
                    vt[2 * KPS + pos] = qn * d;
                    vt[3 * KPS + pos] = d;
                    qk = fmaf(qn, kn, qk);
                }
            }
            qk = WaveSum64(qk);
            if (lane == 0) sQK[buf * TB + tt] = qk;
        }
#pragma unroll
        for (int k = 0; k < WVPT; ++k) {
            const int i = tid + k * THREADS;
            const bool ok = i / COLS < nt && v0 + i % COLS < dv;
            if (i < TB * COLS) sWV[buf * TB * COLS + i] = ok ? rw[k] * rv[k] : 0.0f;   // w * v (reference :120)
        }
    };

    // lane's keys [kb, kb + KT) start at this LDS offset within a vector
    const int kpos = S_::Pos(kb);

    // Recurrence over one block (reference :82-140, one-phase form above).
    auto recur_block = [&](int t0, int buf) __attribute__((always_inline)) {
        const float *vb_ = sVec + buf * TB * RS + kpos;
        const float *wvb = sWV + buf * TB * COLS + cl;
        const float *qkb = sQK + buf * TB;
        float cur[4][KT], nxt[4][KT];
        float cwv, nwv = 0.0f, cqk, nqk = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; ++m) LoadKeys<KT>(vb_ + m * KPS, cur[m]);
        cwv = wvb[0];
        cqk = qkb[0];
        float oreg = 0.0f;
#pragma unroll
        for (int tt = 0; tt < TB; ++tt) {
            if (tt + 1 < TB) {
#pragma unroll
                for (int m = 0; m < 4; ++m) LoadKeys<KT>(vb_ + (tt + 1) * RS + m * KPS, nxt[m]);
                nwv = wvb[(tt + 1) * COLS];
                nqk = qkb[tt + 1];
            }
            const float (&kn)[KT] = cur[0];
            const float (&bkd)[KT] = cur[1];
            const float (&qd)[KT] = cur[2];
            const float (&dec)[KT] = cur[3];
            // e and r are two independent chains; the other wave of the SIMD covers their latency
            float e = 0.0f, r = 0.0f;
#pragma unroll
            for (int j = 0; j < KT; ++j) {
                e = fmaf(bkd[j], S[j], e);
                r = fmaf(qd[j], S[j], r);
            }
            e = ColumnSum<R>(e);
            r = ColumnSum<R>(r);
            const float u = cwv - e;
            const float o = fmaf(cqk, u, r);
#pragma unroll
            for (int j = 0; j < KT; ++j) S[j] = fmaf(kn[j], u, S[j] * dec[j]);
            oreg = kg == tt ? o : oreg;
            if (tt + 1 < TB) {
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int j = 0; j < KT; ++j) cur[m][j] = nxt[m][j];
                cwv = nwv;
                cqk = nqk;
            }
        }
        // lane kg of the column's first row holds the output of token kg of the block
        if (rho == 0 && kg < min(TB, T - t0) && col < dv) p.out[vbase + static_cast<size_t>(t0 + kg) * vstride + col] = oreg;
    };

    if (T > 0) {   // workgroup-uniform: an empty sequence passes its state through
        load_block(0);
        prep_block(0, 0);
        __syncthreads();
        const int nblk = (T + TB - 1) / TB;
        for (int j = 0; j < nblk; ++j) {
            const int buf = j & 1;
            const bool next = j + 1 < nblk;
            if (next) load_block((j + 1) * TB);
            recur_block(j * TB, buf);
            if (next) prep_block((j + 1) * TB, buf ^ 1);
            __syncthreads();
        }
    }
    // State after the last token (identity tokens of a short last block keep it unchanged).
    if (p.final_state != nullptr && col < dv) {
#pragma unroll
        for (int j = 0; j < KT; ++j) {
            const int kd = kb + j;
            if (kd < dk) p.final_state[sbase + static_cast<size_t>(kd) * dv + col] = S[j];
        }
    }
}

// ---------------------------------------------------------------------------
// LDS-state recurrence (dk > 512)
// ---------------------------------------------------------------------------
// GLOBAL: the tile lives in a scratch region of its own (p.state, one
// [dk_pad x 16] tile per (b,h, column block) in the same lane order), which
// also carries it from one token chunk to the next.
template <bool GLOBAL>
__global__ __launch_bounds__(kThreads) void Gdn2RecurLdsKernel(GatedDeltaNet2Params p, int t0, int tc) {
    // State tile: key kd = kg*kt + j of column cl lives at (j*16 + cl)*16 + kg, so
    // the 16 lanes of a row touch 16 consecutive floats (no bank conflicts).
    extern __shared__ __attribute__((aligned(16))) float sLds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int kg = lane & 15, cg = lane >> 4;
    const int cl = w * 4 + cg;                  // column within the workgroup (16 per workgroup)
    const int nvb = (p.dv + 15) / 16;
    const int wg = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int vb = wg % nvb;
    const int bh = wg / nvb;
    const int b = bh / p.nheads, h = bh % p.nheads;
    const int dk = p.dk, dv = p.dv, kp = p.dk_pad;
    const int kt = kp / 16;                     // keys per lane (multiple of 4)
    const int col = vb * 16 + cl;
    const bool col_ok = col < dv;
    const int row = PrepRow(kp);
    float *const sS = GLOBAL ? p.state + static_cast<size_t>(bh * nvb + vb) * kp * 16 : sLds;

    const float *sinit = nullptr;
    if (t0 > 0) sinit = GLOBAL ? nullptr : p.state;   // GLOBAL: the tile already holds the carry
    else if (p.initial_state) sinit = p.initial_state;
    const size_t sbase = static_cast<size_t>(bh) * dk * dv;
    if (!GLOBAL || t0 == 0) {
        for (int j = 0; j < kt; ++j) {
            const int kd = kg * kt + j;
            sS[(j * 16 + cl) * 16 + kg] =
                (sinit && kd < dk && col_ok) ? sinit[sbase + static_cast<size_t>(kd) * dv + col] : 0.0f;
        }
    }
    // Each lane touches only its own (key, column) cells: no barrier needed.

    const float *prep = p.prepared + static_cast<size_t>(bh) * p.chunk_cap * static_cast<size_t>(row);
    for (int tt = 0; tt < tc; ++tt) {
        const float *vt = prep + static_cast<size_t>(tt) * row + kg * kt;
        const size_t vidx = ((static_cast<size_t>(b) * p.seqlen + t0 + tt) * p.nheads + h) * dv + min(col, dv - 1);
        const float wv = col_ok ? p.w[vidx] * p.v[vidx] : 0.0f;
        const float qk = p.prep_qk[static_cast<size_t>(bh) * p.chunk_cap + tt];
        float e = 0.0f, r = 0.0f;
        for (int j = 0; j < kt; j += 4) {
            const float4 b4 = *reinterpret_cast<const float4 *>(vt + kp + j);
            const float4 q4 = *reinterpret_cast<const float4 *>(vt + 2 * kp + j);
            const float bb[4] = {b4.x, b4.y, b4.z, b4.w}, qq[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const float s = sS[((j + x) * 16 + cl) * 16 + kg];
                e = fmaf(bb[x], s, e);
                r = fmaf(qq[x], s, r);
            }
        }
        e = RowSum16(e);
        r = RowSum16(r);
        const float u = wv - e;
        const float o = fmaf(qk, u, r);
        for (int j = 0; j < kt; j += 4) {
            const float4 k4 = *reinterpret_cast<const float4 *>(vt + j);
            const float4 d4 = *reinterpret_cast<const float4 *>(vt + 3 * kp + j);
            const float kk[4] = {k4.x, k4.y, k4.z, k4.w}, dd[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                float &s = sS[((j + x) * 16 + cl) * 16 + kg];
                s = fmaf(kk[x], u, s * dd[x]);
            }
        }
        if (kg == 0 && col_ok) p.out[vidx] = o;
    }
    // carry to the next chunk, or the final state after the last one
    // (GLOBAL: the tile is the carry; only the final state is copied out)
    float *dst = t0 + tc < p.seqlen ? (GLOBAL ? nullptr : p.state) : p.final_state;
    if (dst != nullptr) {
        for (int j = 0; j < kt; ++j) {
            const int kd = kg * kt + j;
            if (kd < dk && col_ok) dst[sbase + static_cast<size_t>(kd) * dv + col] = sS[(j * 16 + cl) * 16 + kg];
        }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
size_t Align256(size_t bytes) { return (bytes + 255) / 256 * 256; }

// Keys per lane for a column of R rows of 16 lanes.
int KeyTile(int dk, int r) {
    const int kt = (dk + 16 * r - 1) / (16 * r);
    for (int c : {1, 2, 4, 6, 8, 12, 16})
        if (kt <= c) return c;
    return 0;
}

int PadKeysLds(int dk) { return (dk + 63) / 64 * 64; }

struct FusedConfig {
    int kt, r, nw;
};

// Rows per column (1, 2 or 4): more rows mean fewer keys per lane and more
// waves, at the price of one or two more reduction steps per sum.  Measured:
// one row wins from one wave per SIMD (1024 waves) up, two rows only from two
// waves per SIMD (2048), else four (at most 8 keys per lane).  8-wave
// workgroups when they still give one workgroup per CU, else 4-wave ones.
// The gdn2_rows override (1, 2 or 4) forces the rows per column where the keys fit, for
// tuning and tests.
FusedConfig ChooseFused(const GatedDeltaNet2Params &p) {
    const long long cols = static_cast<long long>(p.batch) * p.nheads * p.dv;
    const int forced = static_cast<int>(GetOverride(kOverrideGdn2Rows));
    FusedConfig best{0, 0, 8};
    for (int r : {1, 2, 4}) {
        const int kt = KeyTile(p.dk, r);
        if (kt == 0 || (r == 4 && kt > 8)) continue;
        best.kt = kt;
        best.r = r;
        if (r == forced) break;
        if (forced == 0 && cols * r / 4 >= (r == 1 ? 1024 : 2048)) break;
    }
    const long long wgs8 = static_cast<long long>(p.batch) * p.nheads * ((p.dv + 32 / best.r - 1) / (32 / best.r));
    best.nw = wgs8 >= 256 ? 8 : 4;
    return best;
}

template <int KT, int NW, int R>
void LaunchFused(const GatedDeltaNet2Params &p, hipStream_t stream) {
    using L = FusedLayout<KT, NW, R>;
    const long long blocks = static_cast<long long>(p.batch) * p.nheads * ((p.dv + L::COLS - 1) / L::COLS);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    EnsureDynamicLds(reinterpret_cast<const void *>(&Gdn2FusedKernel<KT, NW, R>), static_cast<int>(L::kBytes));
    XM_NOTE_LAUNCH("Gdn2FusedKernel", {}, KT, NW, R);
    hipLaunchKernelGGL((Gdn2FusedKernel<KT, NW, R>), dim3(static_cast<unsigned>(blocks)), dim3(L::THREADS), L::kBytes,
                       stream, p);
}

template <int NW, int R>
void LaunchFusedNR(const GatedDeltaNet2Params &p, int kt, hipStream_t stream) {
    switch (kt) {
        case 1: LaunchFused<1, NW, R>(p, stream); break;
        case 2: LaunchFused<2, NW, R>(p, stream); break;
        case 4: LaunchFused<4, NW, R>(p, stream); break;
        case 6: LaunchFused<6, NW, R>(p, stream); break;
        case 8: LaunchFused<8, NW, R>(p, stream); break;
        default:
            if constexpr (R < 4) {
                if (kt == 12) LaunchFused<12, NW, R>(p, stream);
                else LaunchFused<16, NW, R>(p, stream);
            }
            break;
    }
}

template <int NW>
void LaunchFusedN(const GatedDeltaNet2Params &p, const FusedConfig &c, hipStream_t stream) {
    if (c.r == 1) LaunchFusedNR<NW, 1>(p, c.kt, stream);
    else if (c.r == 2) LaunchFusedNR<NW, 2>(p, c.kt, stream);
    else LaunchFusedNR<NW, 4>(p, c.kt, stream);
}

template <int KPL>
void LaunchPrep(const GatedDeltaNet2Params &p, int t0, int tc, hipStream_t stream) {
    const long long rows = static_cast<long long>(p.batch) * p.nheads * tc;
    const long long blocks = (rows + 3) / 4;
    XM_NOTE_LAUNCH("Gdn2PrepKernel", {}, KPL);
    hipLaunchKernelGGL((Gdn2PrepKernel<KPL>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream, p, t0, tc);
}

void Prep(const GatedDeltaNet2Params &p, int t0, int tc, hipStream_t stream) {
    const int kpl = (p.dk_pad + 63) / 64;
    if (kpl <= 4) LaunchPrep<4>(p, t0, tc, stream);
    else if (kpl <= 8) LaunchPrep<8>(p, t0, tc, stream);
    else if (kpl <= 16) LaunchPrep<16>(p, t0, tc, stream);
    else if (kpl <= 32) LaunchPrep<32>(p, t0, tc, stream);
    else {
        const long long blocks = (static_cast<long long>(p.batch) * p.nheads * tc + 3) / 4;
        XM_NOTE_LAUNCH("Gdn2PrepLoopKernel", {}, );
        hipLaunchKernelGGL(Gdn2PrepLoopKernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream, p, t0,
                           tc);
    }
}

// Scratch of the dk > 512 path for a budget of `cap` bytes: tokens per
// preparation chunk (at most 1024, fewer when the budget is smaller) and the
// regions, each 256-byte aligned: prepared vectors | qhat.khat per row | state.
// The state region is the carry between chunks ([B,H,dk,dv], only when the
// sequence spans several chunks), or above 2048 keys the recurrence's own tile
// store ([B*H*column blocks][dk_pad x 16]).
struct LdsPlan {
    int chunk_cap = 0;     // 0: the budget cannot hold one token
    bool global_state = false;
    size_t prep = 0, qk = 0, state = 0;
    size_t total() const { return prep + qk + state; }
};

LdsPlan PlanLds(int batch, int seqlen, int nheads, int dk, int dv, size_t cap) {
    LdsPlan l;
    const size_t bh = static_cast<size_t>(batch) * nheads;
    const size_t kp = static_cast<size_t>(PadKeysLds(dk));
    l.global_state = kp > static_cast<size_t>(kMaxLdsKeys);
    const size_t tile_store = Align256(bh * ((dv + 15) / 16) * kp * 16 * sizeof(float));
    const size_t carry = Align256(bh * dk * dv * sizeof(float));
    const size_t per_token = bh * (PrepRow(static_cast<int>(kp)) + 1) * sizeof(float);
    auto fill = [&](int c) {
        l.chunk_cap = c;
        l.prep = Align256(bh * c * PrepRow(static_cast<int>(kp)) * sizeof(float));
        l.qk = Align256(bh * c * sizeof(float));
        l.state = l.global_state ? tile_store : (c < seqlen ? carry : 0);
    };
    fill(std::min(seqlen, kChunkTokens));
    if (l.total() <= cap) return l;
    // a shorter chunk: the state region is then always needed
    const size_t state = l.global_state ? tile_store : carry;
    const size_t room = cap > state + 512 ? cap - state - 512 : 0;   // 512: the two alignment pads
    const int c = static_cast<int>(std::min<size_t>(room / per_token, static_cast<size_t>(kChunkTokens)));
    if (c < 1) {
        l.chunk_cap = 0;
        return l;
    }
    fill(c);
    return l;
}

}  // namespace

size_t GatedDeltaNet2ScratchBytes(int batch, int seqlen, int nheads, int dk, int dv, bool packed, size_t cap,
                                  bool allow_split) {
    if (dk <= kGdn2ChunkKeyLimit && GetOverride(kOverrideGdn2Path) != 1)   // chunked path (packed included)
        return GatedDeltaNet2ChunkScratchBytes(batch, seqlen, nheads, dk, dv, packed, cap, allow_split);
    if (dk <= kFusedKeyLimit) return 0;   // fused kernel: no scratch
    const LdsPlan l = PlanLds(batch, seqlen, nheads, dk, dv, cap);
    return l.chunk_cap == 0 ? SIZE_MAX : l.total();
}

void LaunchGatedDeltaNet2(GatedDeltaNet2Params p, void *scratch, size_t scratch_bytes, void *stream_v) {
    // packed: token rows outside every sequence are zeros, not left unwritten
    if (p.cu_seqlens != nullptr)
        LaunchPackedGaps(p.out, static_cast<size_t>(p.nheads) * p.dv, p.cu_seqlens, p.batch, p.seqlen, stream_v);
    // dk <= 512: gated_deltanet2_chunk.hip (the fused kernel under the gdn2_path override)
    if (LaunchGatedDeltaNet2Chunked(p, scratch, scratch_bytes, stream_v)) return;
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    if (p.cu_seqlens != nullptr && p.dk > kFusedKeyLimit)
        throw Error(XM_ERR_UNSUPPORTED, "GatedDeltaNet2Fn with cu_seqlens supports headdim_k up to 512");
    if (p.dk <= kFusedKeyLimit) {
        const FusedConfig c = ChooseFused(p);
        if (c.nw == 8) LaunchFusedN<8>(p, c, stream);
        else LaunchFusedN<4>(p, c, stream);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn");
        return;
    }
    // dk > 512: preparation in token chunks, state in LDS (or above 2048 keys in
    // a scratch region of its own), carried through scratch
    const LdsPlan l = PlanLds(p.batch, p.seqlen, p.nheads, p.dk, p.dv, scratch_bytes);
    if (l.chunk_cap == 0 || l.total() > scratch_bytes || (l.total() > 0 && scratch == nullptr))
        throw Error(XM_ERR_ALLOC, "GatedDeltaNet2Fn: the scratch buffer is smaller than the call needs");
    p.dk_pad = PadKeysLds(p.dk);
    p.chunk_cap = l.chunk_cap;
    char *base = static_cast<char *>(scratch);
    p.prepared = reinterpret_cast<float *>(base);
    p.prep_qk = reinterpret_cast<float *>(base + l.prep);
    p.state = l.state > 0 ? reinterpret_cast<float *>(base + l.prep + l.qk) : nullptr;
    const long long bh = static_cast<long long>(p.batch) * p.nheads;
    if (bh * ((p.dv + 15) / 16) > 2147483647LL || (bh * p.chunk_cap + 3) / 4 > 2147483647LL)
        throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    const size_t lds = l.global_state ? 0 : static_cast<size_t>(p.dk_pad) * 16 * sizeof(float);
    if (!l.global_state) EnsureDynamicLds(reinterpret_cast<const void *>(&Gdn2RecurLdsKernel<false>), static_cast<int>(lds));
    for (int t0 = 0; t0 < p.seqlen; t0 += p.chunk_cap) {
        const int tc = std::min(p.chunk_cap, p.seqlen - t0);
        Prep(p, t0, tc, stream);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn preparation");
        const long long blocks = bh * ((p.dv + 15) / 16);
        if (l.global_state) {
            XM_NOTE_LAUNCH("Gdn2RecurLdsKernel", {}, 1);
            hipLaunchKernelGGL(Gdn2RecurLdsKernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream,
                               p, t0, tc);
        } else {
            XM_NOTE_LAUNCH("Gdn2RecurLdsKernel", {}, 0);
            hipLaunchKernelGGL(Gdn2RecurLdsKernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds,
                               stream, p, t0, tc);
        }
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn recurrence");
    }
}

}  // namespace xm
