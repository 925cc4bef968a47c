// GatedDeltaNet2Fn forward for gfx950: chunked form on fp32 MFMA (dk <= 256).
//
// The reference recurrence (gated_deltanet2_fwd.cu:82-140), per (b,h), with
// qhat, khat the normalised q, k, d = exp(g), bk = beta*khat, wv = w*v:
//     S_t = diag(d_t) S_{t-1} + khat_t u_t^T,   u_t = wv_t - bk_t^T diag(d_t) S_{t-1},
//     o_t = qhat_t^T S_t.
// Over a chunk of C = 16 tokens that starts from the state S0 this unrolls to
// (G_t = prod_{r<=t} d_r inclusive, P_ts = G_t / G_s = prod_{s<r<=t} d_r):
//     e_t = (bk_t o G_t)^T S0 + sum_{s<t} a_ts u_s,   a_ts  = sum_i bk_ti P_tsi khat_si
//     o_t = (qhat_t o G_t)^T S0 + sum_{s<=t} m_ts u_s, m_ts = sum_i qhat_ti P_tsi khat_si
// so with E = [bk_t o G_t], R = [qhat_t o G_t], Y = WV - E S0 and
// T = (I + A)^-1 (A strictly lower triangular):
//     U = T Y,   O = R S0 + (M T) Y,   S_C = G_15 o S0 + Ut^T U,
// Ut_s = khat_s o prod_{s<r<=15} d_r.  A and M take E and R against
// khat_s / G_s; a chunk whose cumulative decays leave [2^-60, 2^60] (1/G could
// overflow or G underflow) takes the decay products pairwise instead, as
// exp(Lg_t - Lg_s) with Lg the prefix sum of g, and Ut from a suffix product:
// no division.  The tail of the sequence is padded with identity tokens
// (d = 1, zero vectors), which leave the state unchanged.
//
// Two kernels per window of up to 128 chunks (2048 tokens):
//  * Gdn2ChunkPrepKernel: one wave per (b,h,chunk), all chunks in parallel.
//    L2 norms, decay products, E, R, Ut, G_15, A, M (MFMA), T (forward
//    substitution), M T (MFMA), written to scratch in the lane order of the
//    MFMA operands, so the recurrence reads each with one 16-byte load per
//    lane.
//  * Gdn2ChunkRecurKernel: a workgroup owns one (b,h) and CT tiles of 16 value
//    columns; KS waves split the keys of a column tile (KPW tiles of 16 keys
//    per wave), the state of a wave being KPW 16x16 accumulator tiles.  Per
//    chunk: S = G_15 o S + Ut^T U of the previous chunk, partial E S0 and R S0
//    (MFMA), one barrier, the partials summed, U = T Y and O = R S0 + (M T) Y
//    (MFMA), O stored.  The state crosses windows through scratch.
// The matrix products use v_mfma_f32_16x16x4_f32 (A[m][k] in lane m+16k, B[k][n]
// in lane n+16k, D[m][n] in lane n+16(m/4), register m%4); the D layout of the
// state, of Y and of U serves directly as the B operand of the next product.
// Numerics differ from the sequential reference by fp32 rounding only; the
// parity tests bound the difference against the fp64 oracle.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <utility>

#include "xm_hip.h"
#include "xm_params.h"

namespace xm {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kC = 16;                   // tokens per chunk
constexpr int kChunkKeyLimit = 256;     // dk handled by the chunked path
constexpr float kL2EpsC = 1.0e-6f;       // reference kL2NormEps (gated_deltanet2_fwd.cu:14)
constexpr float kDecayLo = 0x1p-60f;     // fast-path range of the cumulative decays
constexpr float kDecayHi = 0x1p60f;
constexpr int kSP = 20;                  // pitch of the 16-wide LDS matrices (odd multiple of 4)
constexpr int kTile = 16 * kSP;          // one 16 x 16 matrix in LDS

__device__ __forceinline__ v4f Mfma(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f LdsF4(const float *p) { return *reinterpret_cast<const v4f *>(p); }
__device__ __forceinline__ void StF4(float *p, v4f v) { *reinterpret_cast<v4f *>(p) = v; }

// Orders this wave's LDS accesses before and after (the LDS unit serves one
// wave's operations in order; this stops the compiler from moving them).
__device__ __forceinline__ void WaveSync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// DPP move within a row of 16 lanes; lanes whose source is outside the row keep `old`.
template <int CTRL>
__device__ __forceinline__ float DppOr(float old, float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Scans over the 16 lanes of each row (the 16 tokens of a chunk), Hillis-Steele.
__device__ __forceinline__ float RowPrefixMul(float x) {   // prod_{j <= m} x_j
    x *= DppOr<0x111>(1.0f, x);   // row_shr:1
    x *= DppOr<0x112>(1.0f, x);   // row_shr:2
    x *= DppOr<0x114>(1.0f, x);   // row_shr:4
    x *= DppOr<0x118>(1.0f, x);   // row_shr:8
    return x;
}
__device__ __forceinline__ float RowPrefixAdd(float x) {   // sum_{j <= m} x_j
    x += DppOr<0x111>(0.0f, x);
    x += DppOr<0x112>(0.0f, x);
    x += DppOr<0x114>(0.0f, x);
    x += DppOr<0x118>(0.0f, x);
    return x;
}
__device__ __forceinline__ float RowSuffixMulExcl(float x) {   // prod_{j > m} x_j
    x *= DppOr<0x101>(1.0f, x);   // row_shl:1
    x *= DppOr<0x102>(1.0f, x);   // row_shl:2
    x *= DppOr<0x104>(1.0f, x);   // row_shl:4
    x *= DppOr<0x108>(1.0f, x);   // row_shl:8
    return DppOr<0x101>(1.0f, x);
}
// Value of lane 15 of this lane's row (DPP row_newbcast:15).
__device__ __forceinline__ float RowLast(float x) { return DppF<0x15F>(x); }
// Sum over the 4 rows at this lane's position in the row (gfx950 lane swaps).
__device__ __forceinline__ float RowsSum4(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}
// Lane m of each row gets lane (m - D) mod 16 of the row.
template <int D>
__device__ __forceinline__ float RowRor(float x) {
    if constexpr (D == 0) return x;
    else return DppF<0x120 + D>(x);
}

constexpr int kWindowChunks = 128;       // chunks per prep/recurrence window (2048 tokens)

size_t Align256(size_t bytes) { return (bytes + 255) / 256 * 256; }
constexpr int kPrepWaves = 4;            // waves (chunk-heads) per prep workgroup

// Chunk-head block of the prepared window, in floats, for kq key tiles.  The
// vectors are unnormalised (q, k in place of qhat, khat); the recurrence
// applies the per-token multipliers to the rows of E S0, R S0 and U.
//   E' = beta k G tiles [kq][256], R' = q G tiles [kq][256]: lane l holds
//     token l%16, keys 4(l/16)..+3 of the tile
//   Ut' tiles [kq][256] (k prod_{r>t} d_r): lane l holds key l%16, tokens 4(l/16)..+3
//   G_15 [kq][16]; T [256], M T [256]: lane l holds row l%16, columns 4(l/16)..+3
//   q and k multipliers [2][16]
__host__ __device__ constexpr int BlockFloats(int kq) { return 3 * kq * 256 + 16 * kq + 512 + 32; }

__device__ __forceinline__ v4f LdgF4(const float *p) { return *reinterpret_cast<const v4f *>(p); }
__device__ __forceinline__ void StgF4(float *p, v4f v) { *reinterpret_cast<v4f *>(p) = v; }

// Raw inputs of one key tile of one chunk in operand layout (lane m + 16g:
// token t0 + m, keys kt*16 + 4g + i), zero past the ends.
__device__ __forceinline__ void LoadKeyTile(const GatedDeltaNet2Params &p, size_t rowbase, bool live, int kt,
                                            int g4, float (&q)[4], float (&k)[4], float (&g)[4], float (&bt)[4]) {
    const int k0 = kt * 16 + 4 * g4;
    if (p.vec4_keys) {
        const size_t at = rowbase + min(k0, p.dk - 4);
        const v4f q4 = LdgF4(p.q + at), k4 = LdgF4(p.k + at), g4v = LdgF4(p.g + at), b4 = LdgF4(p.beta + at);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ok = live && k0 + i < p.dk;
            q[i] = ok ? q4[i] : 0.0f;
            k[i] = ok ? k4[i] : 0.0f;
            g[i] = ok ? g4v[i] : 0.0f;
            bt[i] = ok ? b4[i] : 0.0f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ok = live && k0 + i < p.dk;
            const size_t at = rowbase + min(k0 + i, p.dk - 1);
            q[i] = ok ? p.q[at] : 0.0f;
            k[i] = ok ? p.k[at] : 0.0f;
            g[i] = ok ? p.g[at] : 0.0f;
            bt[i] = ok ? p.beta[at] : 0.0f;
        }
    }
}

// One token distance D of the pairwise A and M over all key tiles: lane t of
// each row meets token s = t - D through a row rotation.  Results go to `dst`
// in the D layout of (t, s): [A: 256][M: 256].
template <int D>
__device__ __forceinline__ void PairStep(const GatedDeltaNet2Params &p, size_t rowbase, bool live, int kq, int m16,
                                         int g4, float qm, float km, float *dst) {
    float a = 0.0f, mm = 0.0f;
    for (int kt = 0; kt < kq; ++kt) {
        float q[4], k[4], g[4], bt[4];
        LoadKeyTile(p, rowbase, live, kt, g4, q, k, g, bt);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float kn = k[i] * km;
            const float lg = RowPrefixAdd(g[i]);
            const float ks_ = RowRor<D>(kn);
            const float pd = __expf(lg - RowRor<D>(lg));   // prod_{s<r<=t} d_r
            a = fmaf(bt[i] * kn * pd, ks_, a);
            mm = fmaf(q[i] * qm * pd, ks_, mm);
        }
    }
    a = RowsSum4(a);
    mm = RowsSum4(mm);
    if (g4 == 0 && m16 >= D) {
        const int t = m16, s = m16 - D;
        const int pos = (s + 16 * (t >> 2)) * 4 + (t & 3);
        dst[pos] = a;
        dst[256 + pos] = mm;
    }
}

template <int... Ds>
__device__ __forceinline__ void PairSteps(std::integer_sequence<int, Ds...>, const GatedDeltaNet2Params &p,
                                          size_t rowbase, bool live, int kq, int m16, int g4, float qm, float km,
                                          float *dst) {
    (PairStep<Ds>(p, rowbase, live, kq, m16, g4, qm, km, dst), ...);
}

// A and M of a chunk whose decays leave the fast range (the whole wave calls
// it).  Inlined: a call would give every wave a stack frame and its traffic.
__device__ __forceinline__ void PairwiseAM(const GatedDeltaNet2Params &p, size_t rowbase, bool live, int kq,
                                                     float qm, float km, float *dst) {
    const int lane = threadIdx.x & 63;
    PairSteps(std::make_integer_sequence<int, kC>{}, p, rowbase, live, kq, lane & 15, lane >> 4, qm, km, dst);
}

// ---------------------------------------------------------------------------
// Preparation: one wave per (b,h,chunk) of the window
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64 * kPrepWaves) void Gdn2ChunkPrepKernel(GatedDeltaNet2Params p, int c0, int wn, int kq) {
    __shared__ float sw[kPrepWaves][4][kTile];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int m16 = lane & 15, g4 = lane >> 4;
    const int T = p.seqlen, H = p.nheads;
    const long long item = static_cast<long long>(blockIdx.x) * kPrepWaves + w;
    if (item >= static_cast<long long>(p.batch) * H * wn) return;   // whole wave; no workgroup barrier here
    const int bh = static_cast<int>(item / wn), cw = static_cast<int>(item % wn);
    const int b = bh / H, h = bh % H;
    const int t0 = (c0 + cw) * kC;
    const bool live = t0 + m16 < T;
    const size_t rowbase = ((static_cast<size_t>(b) * T + min(t0 + m16, T - 1)) * H + h) * p.dk;
    float *const blk = p.prepared + static_cast<size_t>(item) * BlockFloats(kq);
    float *const wTr = sw[w][0], *const wA = sw[w][1], *const wT = sw[w][2], *const wTT = sw[w][3];

    // One pass over the key tiles: the unnormalised chunk vectors, the L2
    // norms of token m16, the range of the cumulative decays, and A', M'
    // (unnormalised A and M) on MFMA, used when every decay product is in range.
    float qs = 0.0f, kq2 = 0.0f;
    bool in_range = true;
    v4f al = {0.0f, 0.0f, 0.0f, 0.0f}, mu = al;
    // one key tile: operand-layout vectors to the block, A' and M' accumulated
    auto tile = [&](int kt, const float (&q)[4], const float (&k)[4], const float (&g)[4], const float (&bt)[4])
                    __attribute__((always_inline)) {
        v4f e, r, kb, g15;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qs = fmaf(q[i], q[i], qs);
            kq2 = fmaf(k[i], k[i], kq2);
            const bool ok = live && kt * 16 + 4 * g4 + i < p.dk;
            // exp(g), hardware exp2 (the reference is built with fast math);
            // padded keys and identity tokens decay by 1
            const float d = ok ? __expf(g[i]) : 1.0f;
            const float G = RowPrefixMul(d);                    // G_t
            in_range = in_range && G >= kDecayLo && G <= kDecayHi;
            g15[i] = RowLast(G);
            e[i] = bt[i] * k[i] * G;                            // beta k G
            r[i] = q[i] * G;                                    // q G
            kb[i] = k[i] * __builtin_amdgcn_rcpf(G);            // k / G (fast range only)
            wTr[(4 * g4 + i) * kSP + m16] = k[i] * RowSuffixMulExcl(d);   // k prod_{r>t} d_r, transposed
        }
        WaveSync();
        const v4f utA = LdsF4(wTr + m16 * kSP + 4 * g4);
        WaveSync();
        StgF4(blk + kt * 256 + lane * 4, e);
        StgF4(blk + (kq + kt) * 256 + lane * 4, r);
        StgF4(blk + (2 * kq + kt) * 256 + lane * 4, utA);
        if (m16 == 0) StgF4(blk + 3 * kq * 256 + kt * 16 + 4 * g4, g15);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            al = Mfma(e[ii], kb[ii], al);
            mu = Mfma(r[ii], kb[ii], mu);
        }
    };
    // key tiles in pairs, both loaded before either is used: the two halves of
    // a 128-byte line of each token row are requested together
    for (int kt = 0; kt < kq; kt += 2) {
        float q0[4], k0[4], g0[4], b0[4], q1[4], k1[4], g1[4], b1[4];
        const bool pair = kt + 1 < kq;   // kq is 1 or even
        LoadKeyTile(p, rowbase, live, kt, g4, q0, k0, g0, b0);
        if (pair) LoadKeyTile(p, rowbase, live, kt + 1, g4, q1, k1, g1, b1);
        tile(kt, q0, k0, g0, b0);
        if (pair) tile(kt + 1, q1, k1, g1, b1);
    }
    qs = RowsSum4(qs);
    kq2 = RowsSum4(kq2);
    float qm = p.scale, km = 1.0f;
    if (p.l2norm) {
        // reference :58-62: q_mul = scale * rsqrt(sum + eps); k_mul = rsqrt(sum + eps)
        qm *= rsqrtf(qs + kL2EpsC);
        km = rsqrtf(kq2 + kL2EpsC);
    }
    float *const mul = blk + 3 * kq * 256 + 16 * kq + 512;
    if (g4 == 0) {
        mul[m16] = qm;
        mul[16 + m16] = km;
    }
    if (__all(in_range) && p.pairwise_only == 0) {
        // A[t][s] = k_mul_t k_mul_s A'[t][s], M[t][s] = q_mul_t k_mul_s M'[t][s]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 4 * g4 + i;
            const float kmt = __shfl(km, t), qmt = __shfl(qm, t);
            al[i] *= kmt * km;
            mu[i] *= qmt * km;
        }
    } else {
        PairwiseAM(p, rowbase, live, kq, qm, km, wA);
        WaveSync();
        al = LdsF4(wA + lane * 4);
        mu = LdsF4(wA + 256 + lane * 4);
        WaveSync();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * g4 + i, s = m16;
        al[i] = t > s ? al[i] : 0.0f;
        mu[i] = t >= s ? mu[i] : 0.0f;
    }

    // T = (I + A)^-1 by forward substitution: lane 4c + q holds T[q + 4j][c],
    // j = 0..3; row r sums A[r][s] T[s][c] over the quad's rows s < r (A is
    // zero on and above the diagonal), then lane q = r % 4 keeps it.
#pragma unroll
    for (int i = 0; i < 4; ++i) wA[(4 * g4 + i) * kSP + (m16 & 3) * 4 + (m16 >> 2)] = al[i];   // [r][s%4][s/4]
    WaveSync();
    const int fc = lane >> 2, fq = lane & 3;
    v4f arow[kC];
#pragma unroll
    for (int r = 0; r < kC; ++r) arow[r] = LdsF4(wA + r * kSP + fq * 4);   // A[r][fq + 4j]
    float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < kC; ++r) {
        float part = arow[r][0] * x[0];
        part = fmaf(arow[r][1], x[1], part);
        part = fmaf(arow[r][2], x[2], part);
        part = fmaf(arow[r][3], x[3], part);
        part += DppF<0xB1>(part);   // quad_perm [1,0,3,2]
        part += DppF<0x4E>(part);   // quad_perm [2,3,0,1]
        const float val = (r == fc ? 1.0f : 0.0f) - part;
        if (fq == (r & 3)) x[r >> 2] = val;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        wT[(fq + 4 * j) * kSP + fc] = x[j];    // T row-major
        wTT[fc * kSP + fq + 4 * j] = x[j];     // T^T row-major
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) wTr[(4 * g4 + i) * kSP + m16] = mu[i];   // M row-major
    WaveSync();
    // M T: A[m][k] = M[m][k], B[k][n] = T[k][n]
    const v4f mA = LdsF4(wTr + m16 * kSP + 4 * g4);
    const v4f tB = LdsF4(wTT + m16 * kSP + 4 * g4);
    v4f mt = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) mt = Mfma(mA[ii], tB[ii], mt);
    StgF4(blk + 3 * kq * 256 + 16 * kq + lane * 4, LdsF4(wT + m16 * kSP + 4 * g4));   // T, A operand
    WaveSync();
#pragma unroll
    for (int i = 0; i < 4; ++i) wTr[(4 * g4 + i) * kSP + m16] = mt[i];
    WaveSync();
    StgF4(blk + 3 * kq * 256 + 16 * kq + 256 + lane * 4, LdsF4(wTr + m16 * kSP + 4 * g4));   // M T, A operand
}

// ---------------------------------------------------------------------------
// Recurrence over one window
// ---------------------------------------------------------------------------
template <int KPW, int KS, int CT>
struct RecurLayout {
    static constexpr int NW = KS * CT;
    static constexpr int THREADS = 64 * NW;
    static constexpr int KQ = KPW * KS;
    static constexpr int FB = BlockFloats(KQ);              // one prepared chunk block
    static constexpr int F4 = FB / 4;
    static constexpr int CP = (F4 + THREADS - 1) / THREADS;  // 16-byte copies per thread per block
    // LDS, in floats: [2][FB] staged blocks | [NW][2][256] partial E' S0, R' S0
    static constexpr int oXp = 2 * FB;
    static constexpr int kFloats = oXp + NW * 512;
    static constexpr size_t kBytes = kFloats * sizeof(float);
};

template <int KPW, int KS, int CT>
__global__ __launch_bounds__(64 * KS * CT) void Gdn2ChunkRecurKernel(GatedDeltaNet2Params p, int c0, int wn,
                                                                     const float *s_in, float *s_out) {
    using L = RecurLayout<KPW, KS, CT>;
    constexpr int KQ = L::KQ, FB = L::FB;
    extern __shared__ float smem[];
    float *const sXp = smem + L::oXp;

    const int T = p.seqlen, H = p.nheads, dk = p.dk, dv = p.dv;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ct = w / KS, ks = w % KS;
    const int m16 = lane & 15, g4 = lane >> 4;
    const int VT = (dv + 15) / 16;
    const int ncg = (VT + CT - 1) / CT;
    const int blk = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int bh = blk / ncg, cg = blk % ncg;
    const int b = bh / H, h = bh % H;
    const int vt = cg * CT + ct;
    const bool tile_live = vt < VT;              // wave-uniform
    const int col = vt * 16 + m16;
    const bool col_ok = tile_live && col < dv;
    const int colc = col_ok ? col : 0;
    const size_t sbase = static_cast<size_t>(bh) * dk * dv;
    const float *const prep0 = p.prepared + static_cast<size_t>(bh) * wn * FB;

    v4f S[KPW];
#pragma unroll
    for (int kt = 0; kt < KPW; ++kt) {
        const int kb = (ks * KPW + kt) * 16 + 4 * g4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = kb + i;
            S[kt][i] = (s_in != nullptr && col_ok && key < dk) ? s_in[sbase + static_cast<size_t>(key) * dv + col] : 0.0f;
        }
    }

    // prepared block of chunk cw: global -> registers (two chunks ahead, set
    // cw % 2) -> LDS buffer cw % 2
    v4f stage0[L::CP], stage1[L::CP];
    auto load_block = [&](int cw, v4f (&st)[L::CP]) __attribute__((always_inline)) {
        const float *const bp = prep0 + static_cast<size_t>(cw) * FB;
#pragma unroll
        for (int j = 0; j < L::CP; ++j) {
            const int idx = min(tid + j * L::THREADS, L::F4 - 1);
            st[j] = LdgF4(bp + idx * 4);
        }
    };
    auto store_block = [&](int buf, const v4f (&st)[L::CP]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < L::CP; ++j) {
            const int idx = tid + j * L::THREADS;
            if (idx < L::F4) StF4(smem + buf * FB + idx * 4, st[j]);
        }
    };
    // w, v of one chunk: tokens 4(l/16)+i, this lane's column.  Two sets in
    // turn with compile-time roles (a runtime-indexed pair would make the
    // consumer wait for the newest loads as well).
    struct WV {
        float w[4], v[4];
    };
    auto load_wv = [&](int cw, WV &x) __attribute__((always_inline)) {
        const int t0 = (c0 + cw) * kC;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = min(t0 + 4 * g4 + i, T - 1);
            const size_t idx = ((static_cast<size_t>(b) * T + t) * H + h) * dv + colc;
            x.w[i] = p.w[idx];
            x.v[i] = p.v[idx];
        }
    };
    // block offsets (floats)
    constexpr int oE = 0, oR = KQ * 256, oU = 2 * KQ * 256, oG = 3 * KQ * 256;
    constexpr int oT = oG + 16 * KQ, oMT = oT + 256, oMul = oT + 512;

    v4f u_prev = {0.0f, 0.0f, 0.0f, 0.0f};   // k_mul o U of the previous chunk
    auto update = [&](const float *blkl) __attribute__((always_inline)) {   // S = G_15 o S + Ut'^T u_prev
#pragma unroll
        for (int kt = 0; kt < KPW; ++kt) {
            const int kg = ks * KPW + kt;
            S[kt] *= LdsF4(blkl + oG + kg * 16 + 4 * g4);
            const v4f ua = LdsF4(blkl + oU + kg * 256 + lane * 4);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) S[kt] = Mfma(ua[ii], u_prev[ii], S[kt]);
        }
    };

    load_block(0, stage0);
    store_block(0, stage0);
    load_block(min(1, wn - 1), stage1);
    load_block(min(2, wn - 1), stage0);
    // Loads below are issued on every path (chunk indices clamped to the
    // window, idle column tiles reading column 0): with a load count that
    // depends on the path, the compiler's wait counts turn conservative and a
    // consumer waits for the newest prefetches as well.
    WV wv0, wv1;
    load_wv(0, wv0);
    __syncthreads();
    // one chunk; stage_nx holds chunk cw + 1 and then receives chunk cw + 3;
    // wv_cur holds this chunk's w, v and wv_nx receives chunk cw + 1's
    auto step = [&](int cw, v4f (&stage_nx)[L::CP], const WV &wv_cur, WV &wv_nx) __attribute__((always_inline)) {
        const int t0 = (c0 + cw) * kC;
        load_wv(min(cw + 1, wn - 1), wv_nx);
        const float *const cur = smem + (cw & 1) * FB;
        const float *const prv = smem + ((cw + 1) & 1) * FB;   // chunk cw - 1 (until it is refilled below)
        if (tile_live) {
            if (cw > 0) update(prv);
            v4f xe = {0.0f, 0.0f, 0.0f, 0.0f}, xr = xe;
#pragma unroll
            for (int kt = 0; kt < KPW; ++kt) {
                const int kg = ks * KPW + kt;
                const v4f ea = LdsF4(cur + oE + kg * 256 + lane * 4);
                const v4f ra = LdsF4(cur + oR + kg * 256 + lane * 4);
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    xe = Mfma(ea[ii], S[kt][ii], xe);
                    xr = Mfma(ra[ii], S[kt][ii], xr);
                }
            }
            StF4(sXp + (w * 2 + 0) * 256 + lane * 4, xe);
            StF4(sXp + (w * 2 + 1) * 256 + lane * 4, xr);
        }
        __syncthreads();
        // chunk cw + 1 into the buffer of chunk cw - 1 (read only before the barrier)
        if (cw + 1 < wn) store_block((cw + 1) & 1, stage_nx);
        load_block(min(cw + 3, wn - 1), stage_nx);
        if (tile_live) {
            v4f xe = LdsF4(sXp + ((ct * KS) * 2 + 0) * 256 + lane * 4);
            v4f xr = LdsF4(sXp + ((ct * KS) * 2 + 1) * 256 + lane * 4);
#pragma unroll
            for (int z = 1; z < KS; ++z) {
                xe += LdsF4(sXp + ((ct * KS + z) * 2 + 0) * 256 + lane * 4);
                xr += LdsF4(sXp + ((ct * KS + z) * 2 + 1) * 256 + lane * 4);
            }
            const v4f qm = LdsF4(cur + oMul + 4 * g4);
            const v4f km = LdsF4(cur + oMul + 16 + 4 * g4);
            v4f y;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool ok = col_ok && t0 + 4 * g4 + i < T;
                y[i] = (ok ? wv_cur.w[i] * wv_cur.v[i] : 0.0f) - km[i] * xe[i];   // rows of E' S0 times k_mul
            }
            const v4f ta = LdsF4(cur + oT + lane * 4);
            v4f u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) u = Mfma(ta[ii], y[ii], u);
            u_prev = km * u;   // the update's Ut' is unnormalised
            if (ks == 0) {
                const v4f ma = LdsF4(cur + oMT + lane * 4);
                v4f o = qm * xr;   // rows of R' S0 times q_mul
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) o = Mfma(ma[ii], y[ii], o);
                if (col_ok) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int t = t0 + 4 * g4 + i;
                        if (t < T) p.out[((static_cast<size_t>(b) * T + t) * H + h) * dv + col] = o[i];
                    }
                }
            }
            if (cw == wn - 1) update(cur);   // state after the window
        }
        __syncthreads();
    };
    for (int cw = 0; cw < wn; cw += 2) {
        step(cw, stage1, wv0, wv1);
        if (cw + 1 < wn) step(cw + 1, stage0, wv1, wv0);
    }
    if (s_out != nullptr && col_ok) {
#pragma unroll
        for (int kt = 0; kt < KPW; ++kt) {
            const int kb = (ks * KPW + kt) * 16 + 4 * g4;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (kb + i < dk) s_out[sbase + static_cast<size_t>(kb + i) * dv + col] = S[kt][i];
        }
    }
}

struct ChunkConfig {
    int kpw, ks, ct;
};

// Two key tiles (32 keys) per wave, ks = a power of two waves per column
// tile (keys padded to 32 ks).  Fewer splits leave too few waves for the
// chip (one wave per SIMD at best, and half the SIMDs idle for 4 x 16 heads
// of 128 x 128); more add cross-wave exchanges.  Measured on 4 x 4096 x 16
// heads, dk = dv = 128: ks = 1, 2, 4 -> 1.18, 0.97, 0.93 ms.
ChunkConfig ChooseChunk(int batch, int nheads, int dk, int dv) {
    const int kq = (dk + 15) / 16;
    ChunkConfig c{kq >= 2 ? 2 : 1, 1, 1};
    const int need = (kq + c.kpw - 1) / c.kpw;
    while (c.ks < need) c.ks *= 2;
    const long long heads = static_cast<long long>(batch) * nheads;
    const int vt = (dv + 15) / 16;
    const char *env = std::getenv("XM_GDN2_CT");   // column tiles per workgroup (test switch)
    if (env != nullptr) {
        const int f = std::atoi(env);
        if ((f == 1 || f == 2 || f == 4) && c.ks * f <= 8) c.ct = f;
        return c;
    }
    // one column tile per workgroup when that gives two workgroups per CU
    // (their phases drift apart and overlap); two otherwise, where the keys
    // allow (4 x 16 heads: dv = 128 -> one, 0.93 ms; dv = 65 -> two, 0.85 ms)
    if (heads * vt < 512 && vt >= 2 && c.ks * 2 <= 8) c.ct = 2;
    return c;
}

template <int KPW, int KS, int CT>
void LaunchRecur(const GatedDeltaNet2Params &p, int c0, int wn, int kq, const float *s_in, float *s_out,
                 hipStream_t stream) {
    using L = RecurLayout<KPW, KS, CT>;
    static_assert(L::kBytes <= 160 * 1024, "LDS budget");
    if (kq != L::KQ) throw Error(XM_ERR_DEVICE, "GatedDeltaNet2Fn chunk configuration mismatch");
    const int vt = (p.dv + 15) / 16;
    const long long blocks = static_cast<long long>(p.batch) * p.nheads * ((vt + CT - 1) / CT);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    XM_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&Gdn2ChunkRecurKernel<KPW, KS, CT>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(L::kBytes)));
    hipLaunchKernelGGL((Gdn2ChunkRecurKernel<KPW, KS, CT>), dim3(static_cast<unsigned>(blocks)), dim3(L::THREADS),
                       L::kBytes, stream, p, c0, wn, s_in, s_out);
}

template <int KPW, int KS>
void LaunchRecurCt(const GatedDeltaNet2Params &p, int ct, int c0, int wn, int kq, const float *s_in, float *s_out,
                   hipStream_t stream) {
    if constexpr (KS * 4 <= 8) {
        if (ct == 4) return LaunchRecur<KPW, KS, 4>(p, c0, wn, kq, s_in, s_out, stream);
    }
    if constexpr (KS * 2 <= 8) {
        if (ct == 2) return LaunchRecur<KPW, KS, 2>(p, c0, wn, kq, s_in, s_out, stream);
    }
    LaunchRecur<KPW, KS, 1>(p, c0, wn, kq, s_in, s_out, stream);
}

void LaunchRecurAny(const GatedDeltaNet2Params &p, const ChunkConfig &c, int c0, int wn, int kq, const float *s_in,
                    float *s_out, hipStream_t stream) {
#define XM_GDN2_RECUR(KPW_, KS_) \
    if (c.kpw == KPW_ && c.ks == KS_) return LaunchRecurCt<KPW_, KS_>(p, c.ct, c0, wn, kq, s_in, s_out, stream);
    XM_GDN2_RECUR(1, 1) XM_GDN2_RECUR(2, 1) XM_GDN2_RECUR(2, 2) XM_GDN2_RECUR(2, 4) XM_GDN2_RECUR(2, 8)
#undef XM_GDN2_RECUR
    throw Error(XM_ERR_DEVICE, "GatedDeltaNet2Fn: no chunk kernel for this key tiling");
}

}  // namespace

size_t GatedDeltaNet2ChunkScratchBytes(int batch, int seqlen, int nheads, int dk, int dv) {
    if (dk > kChunkKeyLimit) return 0;
    const ChunkConfig c = ChooseChunk(batch, nheads, dk, dv);
    const int kq = c.kpw * c.ks;
    const int nchunks = (seqlen + kC - 1) / kC;
    const int win = std::min(nchunks, kWindowChunks);
    const size_t heads = static_cast<size_t>(batch) * nheads;
    size_t bytes = Align256(heads * win * BlockFloats(kq) * sizeof(float));
    if (nchunks > kWindowChunks) bytes += Align256(heads * dk * dv * sizeof(float));
    return bytes;
}

bool LaunchGatedDeltaNet2Chunked(const GatedDeltaNet2Params &p, void *scratch, void *stream_v) {
    const char *path = std::getenv("XM_GDN2_PATH");
    if (path != nullptr && std::strcmp(path, "seq") == 0) return false;
    if (p.dk > kChunkKeyLimit) return false;
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    GatedDeltaNet2Params q = p;
    const char *pw = std::getenv("XM_GDN2_PAIRWISE");
    q.pairwise_only = pw != nullptr && std::atoi(pw) != 0;
    auto a16 = [](const void *x) { return (reinterpret_cast<uintptr_t>(x) & 15u) == 0; };
    q.vec4_keys = p.dk % 4 == 0 && a16(p.q) && a16(p.k) && a16(p.g) && a16(p.beta);
    const ChunkConfig c = ChooseChunk(p.batch, p.nheads, p.dk, p.dv);
    const int kq = c.kpw * c.ks;
    const int nchunks = (p.seqlen + kC - 1) / kC;
    const int win = std::min(nchunks, kWindowChunks);
    const size_t heads = static_cast<size_t>(p.batch) * p.nheads;
    char *base = static_cast<char *>(scratch);
    q.prepared = reinterpret_cast<float *>(base);
    base += Align256(heads * win * BlockFloats(kq) * sizeof(float));
    float *const carry = nchunks > kWindowChunks ? reinterpret_cast<float *>(base) : nullptr;
    for (int c0 = 0; c0 < nchunks; c0 += win) {
        const int wn = std::min(win, nchunks - c0);
        const bool first = c0 == 0, last = c0 + wn >= nchunks;
        const long long items = static_cast<long long>(heads) * wn;
        const long long pblocks = (items + kPrepWaves - 1) / kPrepWaves;
        if (pblocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
        hipLaunchKernelGGL(Gdn2ChunkPrepKernel, dim3(static_cast<unsigned>(pblocks)), dim3(64 * kPrepWaves), 0, stream,
                           q, c0, wn, kq);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn chunk preparation");
        LaunchRecurAny(q, c, c0, wn, kq, first ? p.initial_state : carry, last ? p.final_state : carry, stream);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn chunk recurrence");
    }
    return true;
}

}  // namespace xm
