// GatedDeltaNet2Fn forward for gfx950: chunked form on fp32 MFMA (dk <= 512).
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
// Two kernels per window of chunks (128, or more where 128 MiB of prepared
// blocks hold more):
//  * Gdn2ChunkPrepKernel: one wave per (b,h,chunk), all chunks in parallel.
//    L2 norms, decay products, E, R, Ut, G_15, A, M (MFMA), T (forward
//    substitution), M T (MFMA), and Ut~ = T^T Ut (MFMA, so that Ut^T U =
//    Ut~^T Y), written to scratch in the lane order of the MFMA operands, so
//    the recurrence reads each with one 16-byte load per lane.
//  * Gdn2ChunkRecurKernel: a workgroup owns one (b,h) and one tile of 16 value
//    columns; KS waves split the keys (KPW tiles of 16 keys per wave), the
//    state of a wave being KPW 16x16 accumulator tiles.  Per chunk: partial
//    E S0 and R S0 (MFMA), one barrier, the partials summed into Y, the update
//    S = G_15 o S + Ut~^T Y, and this wave's part of O = R S0 + (M T) Y, which
//    wave 0 sums and stores after the next chunk's barrier.  U itself is never
//    formed.  The state crosses windows through scratch.
// Launches with few column tiles (few heads) split the sequence instead:
// every segment runs at once, the later ones from a zero state beside
// identity columns that give their transition and output map, and a combine
// and a correction kernel finish the result (Gdn2ChunkSplitKernel below; two
// unequal segments with the second at two column tiles per workgroup in
// Gdn2ChunkSplit2Kernel; the correction in Gdn2SplitCorrectRegKernel).
// The matrix products use v_mfma_f32_16x16x4_f32 (A[m][k] in lane m+16k, B[k][n]
// in lane n+16k, D[m][n] in lane n+16(m/4), register m%4); the D layout of the
// state and of Y serves directly as the B operand of the next product.
// Numerics differ from the sequential reference by fp32 rounding only; the
// parity tests bound the difference against the fp64 oracle.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <utility>

#include "xm_hip.h"
#include "xm_matrix.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr int kC = 16;                   // tokens per chunk
constexpr float kL2EpsC = 1.0e-6f;       // reference kL2NormEps (gated_deltanet2_fwd.cu:14)
constexpr float kDecayLo = 0x1p-60f;     // fast-path range of the cumulative decays
constexpr float kDecayHi = 0x1p60f;
constexpr int kSP = 20;                  // pitch of the 16-wide LDS matrices (odd multiple of 4)
constexpr int kTile = 16 * kSP;          // one 16 x 16 matrix in LDS


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
constexpr int kPrepWaves = 4;            // waves (chunk-heads) per prep workgroup (2 above 128 keys, see LaunchPrep)

// Chunk-head block of the prepared window, in floats, for a recurrence of ks
// waves of kpw key tiles (kq = kpw ks).  The vectors are unnormalised (q, k
// in place of qhat, khat); the recurrence applies the per-token multipliers
// to the rows of E S0 and R S0.
//   E' = beta k G tiles [kq][256], R' = q G tiles [kq][256]: lane l holds
//     token l%16, keys 4(l/16)..+3 of the tile
//   Ut~ = T^T diag(k_mul) Ut' tiles [kq][256] (Ut' = k prod_{r>t} d_r): lane l
//     holds key l%16, tokens 4(l/16)..+3
//   M T [256]: lane l holds row l%16, columns 4(l/16)..+3
//   scalar vectors [ks][ScalarVecs(kpw)][64], one float per lane of recurrence
//     wave w: lane 16 r + n of vector s holds entry e = 16 s + n of the list
//     k_mul(4 r + i), q_mul(4 r + i) (i = 0..3), then G_15 of keys
//     16 (w kpw + kt) + 4 r + i for kt < kpw (kt-major).  The lanes of row r
//     (the D layout's tokens or keys 4 r..4 r+3) read entry e with a DPP
//     row broadcast: one 4-byte load per lane brings what four to eight
//     16-byte loads of 16-lane broadcasts would (a 16-byte load costs the
//     vector memory path about three times a 4-byte one, whatever its
//     addresses).
__host__ __device__ constexpr int ScalarVecs(int kpw) { return (8 + 4 * kpw + 15) / 16; }
__host__ __device__ constexpr int BlockFloats(int kpw, int ks) {
    return 3 * kpw * ks * 256 + 256 + ks * ScalarVecs(kpw) * 64;
}

__device__ __forceinline__ v4f LdgF4(const float *p) { return *reinterpret_cast<const v4f *>(p); }
__device__ __forceinline__ void StgF4(float *p, v4f v) { *reinterpret_cast<v4f *>(p) = v; }

// Raw inputs of one key tile of one chunk in operand layout (lane m + 16g:
// token t0 + m, keys kt*16 + 4g + i), zero past the ends.
// One key tile's q, k, g and beta for this lane (keys 16 kt + 4 g4 + i, the
// token of rowbase) as loaded: addresses clamped into the row, values not yet
// masked, so the loads can be issued well before their use.  VEC4: the
// caller knows that p.vec4_keys holds (no branch between the two forms, whose
// different load counts would make the loop's wait counts conservative).
struct KeyTileRaw {
    v4f q, k, g, b;
};
template <bool VEC4 = false>
__device__ __forceinline__ KeyTileRaw LoadKeyTileRaw(const GatedDeltaNet2Params &p, size_t rowbase, int kt, int g4) {
    const int k0 = kt * 16 + 4 * g4;
    KeyTileRaw r;
    if (VEC4 || p.vec4_keys) {
        const size_t at = rowbase + min(k0, p.dk - 4);
        r.q = LdgF4(p.q + at);
        r.k = LdgF4(p.k + at);
        r.g = LdgF4(p.g + at);
        r.b = LdgF4(p.beta + at);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const size_t at = rowbase + min(k0 + i, p.dk - 1);
            r.q[i] = p.q[at];
            r.k[i] = p.k[at];
            r.g[i] = p.g[at];
            r.b[i] = p.beta[at];
        }
    }
    return r;
}

// Zeros for padded keys and dead tokens.
__device__ __forceinline__ void MaskKeyTile(const KeyTileRaw &r, bool live, int dk, int kt, int g4, float (&q)[4],
                                            float (&k)[4], float (&g)[4], float (&bt)[4]) {
    const int k0 = kt * 16 + 4 * g4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool ok = live && k0 + i < dk;
        q[i] = ok ? r.q[i] : 0.0f;
        k[i] = ok ? r.k[i] : 0.0f;
        g[i] = ok ? r.g[i] : 0.0f;
        bt[i] = ok ? r.b[i] : 0.0f;
    }
}

__device__ __forceinline__ void LoadKeyTile(const GatedDeltaNet2Params &p, size_t rowbase, bool live, int kt,
                                            int g4, float (&q)[4], float (&k)[4], float (&g)[4], float (&bt)[4]) {
    MaskKeyTile(LoadKeyTileRaw(p, rowbase, kt, g4), live, p.dk, kt, g4, q, k, g, bt);
}

// Token distance D of the pairwise A and M for one key element: lane t of
// each row meets token s = t - D through a row rotation.  The decay product
// prod_{s<r<=t} d_r is exp of the window sum w = sum_{t-D<r<=t} g_r, which
// this call extends by g_{t-D+1}: a sum of the D terms themselves, not a
// difference of prefix sums (after a hard reset, say g = -200, two prefix
// sums near -200 differ by a value whose absolute error is ulp(200)/2, a
// relative error of 1e-5 in every later product of the chunk).
template <int D>
__device__ __forceinline__ void PairTerm(float g, float kn, float bk, float qq, float &w, float &a, float &mm) {
    if constexpr (D > 0) w += RowRor<D - 1>(g);
    const float pd = D == 0 ? 1.0f : __expf(w);
    const float ks_ = RowRor<D>(kn);
    a = fmaf(bk * pd, ks_, a);
    mm = fmaf(qq * pd, ks_, mm);
}

template <int... Ds>
__device__ __forceinline__ void PairTerms(std::integer_sequence<int, Ds...>, float g, float kn, float bk, float qq,
                                          float (&a)[kC], float (&mm)[kC]) {
    float w = 0.0f;
    (PairTerm<Ds>(g, kn, bk, qq, w, a[Ds], mm[Ds]), ...);   // D = 0, 1, ..., 15 in turn
}

// A and M of a chunk whose decays leave the fast range (the whole wave calls
// it), every token distance at once over one pass of the key tiles.  Results
// go to `dst` in the D layout of (t, s): [A: 256][M: 256].
__device__ __forceinline__ void PairwiseAM(const GatedDeltaNet2Params &p, size_t rowbase, bool live, int kq,
                                           float qm, float km, float *dst) {
    const int lane = threadIdx.x & 63, m16 = lane & 15, g4 = lane >> 4;
    float a[kC], mm[kC];
#pragma unroll
    for (int d = 0; d < kC; ++d) a[d] = mm[d] = 0.0f;
    for (int kt = 0; kt < kq; ++kt) {
        float q[4], k[4], g[4], bt[4];
        LoadKeyTile(p, rowbase, live, kt, g4, q, k, g, bt);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float kn = k[i] * km;
            PairTerms(std::make_integer_sequence<int, kC>{}, g[i], kn, bt[i] * kn, q[i] * qm, a, mm);
        }
    }
#pragma unroll
    for (int d = 0; d < kC; ++d) {
        const float ad = RowsSum4(a[d]), md = RowsSum4(mm[d]);
        if (g4 == 0 && m16 >= d) {
            const int t = m16, s = m16 - d;
            const int pos = (s + 16 * (t >> 2)) * 4 + (t & 3);
            dst[pos] = ad;
            dst[256 + pos] = md;
        }
    }
}

// Largest b with off[b] <= g (off non-decreasing over [0, n], off[0] = 0 <= g
// < off[n]): the packed sequence that holds global chunk g.
__device__ __forceinline__ int SequenceOfChunk(const int *off, int n, int g) {
    int lo = 0, hi = n;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= g) lo = mid;
        else hi = mid;
    }
    return lo;
}

// Token range [lo, hi) of packed sequence b, clamped to the row.
__device__ __forceinline__ void PackedRange(const GatedDeltaNet2Params &p, int b, size_t &tok0, int &T) {
    const long long lo = min(max(p.cu_seqlens[b], 0LL), static_cast<long long>(p.seqlen));
    const long long hi = min(max(p.cu_seqlens[b + 1], lo), static_cast<long long>(p.seqlen));
    tok0 = static_cast<size_t>(lo);
    T = static_cast<int>(hi - lo);
}

// ---------------------------------------------------------------------------
// Preparation: one wave per (b,h,chunk) of the window
// ---------------------------------------------------------------------------
// PW waves (chunk-heads) per workgroup.
// Dynamic LDS: PW * kq * 256 floats, each wave's transposed Ut' tiles
// kept until T is known.  kpw, ks: the recurrence's key tiles per wave and
// waves (kq = kpw ks key tiles), which order the scalar vectors.
// AHEAD: each pair of key tiles' loads issued one pair early, before the
// previous pair's work (32 more VGPRs; 16-byte key loads only, p.vec4_keys);
// the arithmetic is the same.
constexpr int kMaxKeyTiles = 32;         // key tiles of the chunked path (dk <= 512)
template <bool AHEAD, int PW>
__global__ __launch_bounds__(64 * PW) void Gdn2ChunkPrepKernel(GatedDeltaNet2Params p, int c0, int wn, int kpw, int ks) {
    __shared__ __attribute__((aligned(16))) float sw[PW][4][kTile];
    extern __shared__ float prep_dyn[];
    const int kq = kpw * ks;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int m16 = lane & 15, g4 = lane >> 4;
    const int H = p.nheads;
    // rows of the window's blocks: (b, h), or h alone for packed sequences,
    // whose window holds chunks [c0, c0 + W) of every sequence, sequence b's at
    // blocks [chunk_off[b], chunk_off[b + 1]) of the row
    const bool packed = p.chunk_off != nullptr;
    const long long rows = packed ? H : static_cast<long long>(p.batch) * H;
    const long long item = static_cast<long long>(blockIdx.x) * PW + w;
    if (item >= rows * wn) return;   // whole wave; no workgroup barrier here
    const int row = static_cast<int>(item / wn), cw = static_cast<int>(item % wn);
    int h, T, t0;
    size_t tok0;
    if (!packed) {
        const int b = row / H;
        h = row % H;
        T = p.seqlen;
        tok0 = static_cast<size_t>(b) * T;
        t0 = (c0 + cw) * kC;
    } else {
        h = row;
        if (cw >= p.chunk_off[p.batch]) return;   // past the window's blocks: never read
        const int b = SequenceOfChunk(p.chunk_off, p.batch, cw);
        PackedRange(p, b, tok0, T);
        t0 = (c0 + cw - p.chunk_off[b]) * kC;
    }
    const bool live = t0 + m16 < T;
    const size_t rowbase = ((tok0 + min(t0 + m16, T - 1)) * H + h) * p.dk;
    float *const blk = p.prepared + static_cast<size_t>(item) * BlockFloats(kpw, ks);
    float *const wTr = sw[w][0], *const wA = sw[w][1], *const wT = sw[w][2], *const wTT = sw[w][3];
    // G_15 of each key, kept until the scalar vectors are written (in wT and
    // wTT, which T takes over afterwards: 2 kTile >= kMaxKeyTiles * 16)
    float *const gsw = wT;
    static_assert(2 * kTile >= kMaxKeyTiles * 16, "G_15 stash");

    // One pass over the key tiles: the unnormalised chunk vectors, the L2
    // norms of token m16, the range of the cumulative decays, and A', M'
    // (unnormalised A and M) on MFMA, used when every decay product is in range.
    float qs = 0.0f, kq2 = 0.0f;
    bool in_range = true;
    // A' and M' are sums over the keys of unnormalised k.k and q.k products,
    // and they carry most of the chunked form's rounding error (the diagonal
    // of M meets each token's own update).  The MFMA adds its four products to
    // the accumulator one fused multiply-add at a time, so a single chain over
    // dk keys would be a dk-step rounding chain.  Blocked instead: a pair of
    // key tiles accumulates from zero in two chains of 16 keys (k-step parity),
    // and the pair's sum is added to the running total once the next pair's
    // loads are issued (added right after its own products, the wait for them
    // delayed those loads: 1.7% at 256 keys): about 17 + dk/32 rounding steps
    // for any dk.
    const v4f z4 = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f al = z4, mu = z4;                     // totals over the key-tile pairs
    v4f alc[2] = {z4, z4}, muc[2] = {z4, z4};  // the current pair's chains
    // this wave's Ut' tiles: lane l holds key l%16, tokens 4(l/16)..+3 (each
    // lane reads back only its own 16 bytes)
    float *const ut = prep_dyn + static_cast<size_t>(w) * kq * 256 + lane * 4;
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
        StF4(ut + kt * 256, utA);
        StgF4(blk + kt * 256 + lane * 4, e);
        StgF4(blk + (kq + kt) * 256 + lane * 4, r);
        if (m16 == 0) StF4(gsw + kt * 16 + 4 * g4, g15);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            alc[ii & 1] = Mfma(e[ii], kb[ii], alc[ii & 1]);
            muc[ii & 1] = Mfma(r[ii], kb[ii], muc[ii & 1]);
        }
    };
    // key tiles in pairs, both loaded before either is used: the two halves of
    // a 128-byte line of each token row are requested together
    // (AHEAD: raw values carried over, masked at their use, so that no select
    // waits for them early)
    // and issued on every pass, past the last pair too (key addresses are
    // clamped into the token's row), so the loop's wait counts are exact)
    KeyTileRaw cur[2], nxt[2];
    auto load_pair = [&](int kt, KeyTileRaw (&x)[2]) __attribute__((always_inline)) {
        x[0] = LoadKeyTileRaw<AHEAD>(p, rowbase, kt, g4);
        if (AHEAD || kt + 1 < kq) x[1] = LoadKeyTileRaw<AHEAD>(p, rowbase, kt + 1, g4);
    };
    if (AHEAD) load_pair(0, cur);
    for (int kt = 0; kt < kq; kt += 2) {
        const bool pair = kt + 1 < kq;   // kq is 1 or even (AHEAD: even)
        if (!AHEAD) load_pair(kt, cur);
        else load_pair(kt + 2, nxt);
        float q0[4], k0[4], g0[4], b0[4], q1[4], k1[4], g1[4], b1[4];
        MaskKeyTile(cur[0], live, p.dk, kt, g4, q0, k0, g0, b0);
        if (pair) MaskKeyTile(cur[1], live, p.dk, kt + 1, g4, q1, k1, g1, b1);
        al += alc[0] + alc[1];   // the previous pair (zeros at the first)
        mu += muc[0] + muc[1];
        alc[0] = alc[1] = muc[0] = muc[1] = z4;
        tile(kt, q0, k0, g0, b0);
        if (pair) tile(kt + 1, q1, k1, g1, b1);
        if (AHEAD) {
            cur[0] = nxt[0];
            cur[1] = nxt[1];
        }
    }
    al += alc[0] + alc[1];
    mu += muc[0] + muc[1];
    qs = RowsSum4(qs);
    kq2 = RowsSum4(kq2);
    float qm = p.scale, km = 1.0f;
    if (p.l2norm) {
        // reference :58-62: q_mul = scale * rsqrt(sum + eps); k_mul = rsqrt(sum + eps)
        qm *= rsqrtf(qs + kL2EpsC);
        km = rsqrtf(kq2 + kL2EpsC);
    }

    // The scalar vectors (see BlockFloats): lane 16 r + n of vector s of
    // recurrence wave v holds entry e = 16 s + n of row r's list.  Written
    // before the pairwise products and T overwrite the G_15 stash.
    WaveSync();
    {
        const int tok = 4 * g4 + (m16 & 3);   // entries e < 8: token 4 r + e % 4
        const float kmt = __shfl(km, tok), qmt = __shfl(qm, tok);
        const int nsv = ScalarVecs(kpw);
        float *const sv = blk + 3 * kq * 256 + 256;
        for (int v = 0; v < ks; ++v) {
            for (int sx = 0; sx < nsv; ++sx) {
                const int e = 16 * sx + m16;
                float val = e < 4 ? kmt : e < 8 ? qmt : 0.0f;
                if (e >= 8 && e < 8 + 4 * kpw) val = gsw[(v * kpw + (e - 8) / 4) * 16 + 4 * g4 + (e & 3)];
                sv[(v * nsv + sx) * 64 + lane] = val;
            }
        }
    }
    WaveSync();
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
    WaveSync();
#pragma unroll
    for (int i = 0; i < 4; ++i) wTr[(4 * g4 + i) * kSP + m16] = mt[i];
    WaveSync();
    StgF4(blk + 3 * kq * 256 + lane * 4, LdsF4(wTr + m16 * kSP + 4 * g4));   // M T, A operand

    // The update S_C = G_15 o S0 + Ut'^T diag(k_mul) U with U = T Y is
    // Ut~^T Y, Ut~ = T^T diag(k_mul) Ut': the recurrence updates from Y and
    // never forms U.  D[s][key] = sum_t T[t][s] k_mul_t Ut'[t][key] on MFMA:
    // A[s][t] = T^T (tB, lane s + 16k holds T[4k + ii][s]), B[t][key] = the
    // Ut' tile scaled per token; the D layout (key l%16, tokens 4(l/16)+i) is
    // the recurrence's A operand.
    v4f km4;   // k_mul of tokens 4 g4 + ii (every row of lanes holds its token's k_mul)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) km4[ii] = __shfl(km, 4 * g4 + ii);
    for (int kt = 0; kt < kq; ++kt) {
        const v4f b = LdsF4(ut + kt * 256) * km4;
        v4f d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) d = Mfma(tB[ii], b[ii], d);
        StgF4(blk + (2 * kq + kt) * 256 + lane * 4, d);
    }
}

// ---------------------------------------------------------------------------
// Recurrence over one window
// ---------------------------------------------------------------------------
// A recurrence workgroup: KS waves of KPW key tiles over CT tiles of 16
// value columns.
template <int KPW, int KS, int CT = 1>
struct RecurLayout {
    static constexpr int THREADS = 64 * KS;
    static constexpr int KQ = KPW * KS;
    static constexpr int FB = BlockFloats(KPW, KS);   // one prepared chunk block
    static constexpr int NSV = ScalarVecs(KPW);        // scalar vectors per wave
    // Token rows i (the D layout's registers) whose w, v a wave loads and
    // whose (M T) Y slice it forms: i = ks + m KS, m < NM (i < 4).
    static constexpr int NM = (4 + KS - 1) / KS;
    // LDS, in floats, per chunk parity: [KS waves][E' S0, output][CT][256]
    // partials, then W o V [CT][256] (lane l: rows 4(l/16)..+3, column l%16)
    // and [256] where the waves without a row write (no branch)
    static constexpr int kPart = KS * 2 * CT * 256 + CT * 256 + 256;
    static constexpr int kFloats = KS > 1 ? 2 * kPart : 1;
};

// The operands of one chunk that a wave needs, in MFMA lane order: its key
// tiles of E', R', Ut~, its scalar vectors (k_mul, q_mul, G_15), and for its
// token rows i = ks + m KS the M T slice (A operand column 4(l/16)+i) and
// this lane's w, v (token 4(l/16)+i) in each of its CT column tiles.
template <int KPW, int KS, int CT>
struct ChunkOperands {
    using L = RecurLayout<KPW, KS, CT>;
    v4f e[KPW], r[KPW], ut[KPW];
    float sc[L::NSV];
    float mt[L::NM], w[CT][L::NM], v[CT][L::NM];
};

// Entry E of a wave's scalar list for the lanes of each row (DPP row_newbcast).
template <int E, int NSV>
__device__ __forceinline__ float ScalarEntry(const float (&sc)[NSV]) {
    static_assert(E / 16 < NSV, "scalar entry beyond the wave's vectors");
    return DppF<0x150 + E % 16>(sc[E / 16]);
}
template <int I, int NSV>
__device__ __forceinline__ float KMul(const float (&sc)[NSV]) { return ScalarEntry<I, NSV>(sc); }
template <int I, int NSV>
__device__ __forceinline__ float QMul(const float (&sc)[NSV]) { return ScalarEntry<4 + I, NSV>(sc); }
template <int KT, int I, int NSV>
__device__ __forceinline__ float G15(const float (&sc)[NSV]) { return ScalarEntry<8 + 4 * KT + I, NSV>(sc); }
template <int NSV>
__device__ __forceinline__ v4f KMulRows(const float (&sc)[NSV]) {
    return v4f{KMul<0, NSV>(sc), KMul<1, NSV>(sc), KMul<2, NSV>(sc), KMul<3, NSV>(sc)};
}
template <int NSV>
__device__ __forceinline__ v4f QMulRows(const float (&sc)[NSV]) {
    return v4f{QMul<0, NSV>(sc), QMul<1, NSV>(sc), QMul<2, NSV>(sc), QMul<3, NSV>(sc)};
}
// S[kt] = G_15 o S[kt] (keys 16 (ks KPW + kt) + 4 (l/16) + i in register i)
template <int KPW, int NSV, int... KT>
__device__ __forceinline__ void DecayState(v4f (&S)[KPW], const float (&sc)[NSV], std::integer_sequence<int, KT...>) {
    ((S[KT] *= v4f{G15<KT, 0, NSV>(sc), G15<KT, 1, NSV>(sc), G15<KT, 2, NSV>(sc), G15<KT, 3, NSV>(sc)}), ...);
}

// One (b,h) row's chunks [cs, cs + nrun) of its sequence, whose prepared
// blocks sit at window-local indices [cw0, cw0 + nrun) of `prep_row` (the row's
// wn blocks of the window).  tok0: the sequence's first token in the [B*T]
// token rows; T: its length; sbase: the row's offset in the [B,H,K,V] states.
// The state comes from s_in (zeros when null) and goes to s_out (not written
// when null).  Every wave of the workgroup calls it with the same arguments.
// Column tiles of a sequence-split run (Gdn2ChunkSplitKernel,
// Gdn2ChunkSplit2Kernel), in units of the workgroup's CT tiles: with VW =
// ceil(VT / CT), units below VW are value columns; unit VW + j carries the
// identity columns 16 (CT j + c)..+15 (keys) in its tile c: WV = 0, initial
// state I, the output goes to `psi` ([B,T,H,KP] rows, KP = keys padded to
// 16) and the final state to a [K][KP] transition.  The padded columns start
// at zero and stay zero, so they are stored as zeros; identity tiles past KP
// (the second tile of the last unit when ceil(dk / 16) is odd) store nothing.
struct SplitTile {
    int tile;
    bool ident;
    float *psi;
};

template <int KPW, int KS, int CT = 1, bool SPLIT = false>
__device__ __forceinline__ void Gdn2RecurRun(const GatedDeltaNet2Params &p, float *sXp, int h, size_t tok0, int T,
                                             int cs, int cw0, int nrun, int wn, const float *prep_row, size_t sbase,
                                             const float *s_in, float *s_out, SplitTile st = {}) {
    using L = RecurLayout<KPW, KS, CT>;
    using Ops = ChunkOperands<KPW, KS, CT>;
    constexpr int KQ = L::KQ, FB = L::FB, NSV = L::NSV, NM = L::NM;
    constexpr int oE = 0, oR = KQ * 256, oU = 2 * KQ * 256, oMT = 3 * KQ * 256, oSc = oMT + 256;   // block offsets (floats)

    const int H = p.nheads, dk = p.dk, dv = p.dv;
    const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4;
    const int VT = (dv + 15) / 16, VW = (VT + CT - 1) / CT;   // column tiles; workgroups per (b, h)
    const int vt = SPLIT ? st.tile : XcdLocalBlock(blockIdx.x, gridDim.x) % VW;
    const bool ident = SPLIT && st.ident;
    // this lane's value column in each of the workgroup's CT column tiles
    int col[CT];
    bool col_ok[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) {
        col[c] = (vt * CT + c) * 16 + (lane & 15);
        col_ok[c] = !ident && col[c] < dv;
    }
    // output column of each tile: the value column, or (identity tile) the
    // key it starts as
    const int OW = ident ? (dk + 15) / 16 * 16 : dv;   // output row width
    int kcol[CT], ocol[CT];
    bool ocol_ok[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) {
        kcol[c] = SPLIT ? ((vt - VW) * CT + c) * 16 + (lane & 15) : 0;
        ocol[c] = ident ? kcol[c] : col[c];
        ocol_ok[c] = ident ? kcol[c] < OW : col_ok[c];
    }
    const Rsrc rblk = MakeRsrc(prep_row, wn * FB * 4);   // this head row's prepared blocks of the window
    // byte offsets, from a chunk's first token in [B,T,H,V], of this lane's
    // tokens 4(l/16)+i in its columns (out of range for columns past dv); the
    // per-chunk descriptors of w, v and out end after the chunk's last valid
    // token, so padded tokens read zeros and are not stored
    const int HV = H * dv;
    int vo[CT][4];
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) vo[c][i] = col_ok[c] ? ((4 * g4 + i) * HV + col[c]) * 4 : kOutOfRange;
    // this wave's token rows i = ks + m KS (clamped to 3 where m KS + ks >= 4,
    // loaded but unused): w, v offsets and the M T slice of the A operand
    int vl[CT][NM], mo[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const int i = min(ks + m * KS, 3);
#pragma unroll
        for (int c = 0; c < CT; ++c) vl[c][m] = col_ok[c] ? ((4 * g4 + i) * HV + col[c]) * 4 : kOutOfRange;
        mo[m] = (lane * 4 + i) * 4;
    }
    const int so = lane * 4 + ks * NSV * 256;   // this wave's scalar vectors
    // Chunk jl of the run starts kC * HV floats after chunk jl - 1 in w, v and
    // out: the run's first rows are formed once, a chunk adds its offset (no
    // 64-bit index arithmetic per chunk).  A chunk's rows end after its last
    // valid token.
    auto token_base = [&](const float *x, int t0) { return x + ((tok0 + t0) * H + h) * dv; };
    const float *const w_run = token_base(p.w, cs * kC);
    const float *const v_run = token_base(p.v, cs * kC);
    const int cstride = kC * HV;
    const int full_bytes = ((kC - 1) * HV + dv) * 4;
    auto rows_bytes = [&](int jl) {
        const int left = T - (cs + jl) * kC;
        return left >= kC ? full_bytes : ((left - 1) * HV + dv) * 4;
    };
    auto chunk_off = [&](int jl) { return static_cast<long long>(jl) * cstride; };
    // the output rows (O, or psi for an identity tile: rows of OW floats)
    const int HO = H * OW;
    int oo[CT][4];
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            oo[c][i] = SPLIT ? (ocol_ok[c] ? ((4 * g4 + i) * HO + ocol[c]) * 4 : kOutOfRange) : vo[c][i];
    // this wave's output rows i = ks + m KS (kOutOfRange for i >= 4: the
    // store is dropped)
    int ol[CT][NM];
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const int i = ks + m * KS;
            const bool ok = i < 4 && ocol_ok[c];
            ol[c][m] = ok ? ((4 * g4 + i) * HO + ocol[c]) * 4 : kOutOfRange;
        }
    float *const out_run = (ident ? st.psi : p.out) + ((tok0 + cs * kC) * H + h) * OW;
    auto out_bytes = [&](int jl) {
        if constexpr (!SPLIT) return rows_bytes(jl);
        const int left = min(T - (cs + jl) * kC, kC);
        return ((left - 1) * HO + OW) * 4;
    };
    auto out_off = [&](int jl) { return static_cast<long long>(jl) * (kC * HO); };

    v4f S[CT][KPW];
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int kt = 0; kt < KPW; ++kt) {
            const int kb = (ks * KPW + kt) * 16 + 4 * g4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kb + i;
                S[c][kt][i] = ident ? (key == kcol[c] && key < dk ? 1.0f : 0.0f)
                                    : (s_in != nullptr && col_ok[c] && key < dk)
                                          ? s_in[sbase + static_cast<size_t>(key) * dv + col[c]]
                                          : 0.0f;
            }
        }

    if (nrun > 0) {   // workgroup-uniform
        // Loads are issued on every path (chunk indices clamped to the range):
        // with a load count that depends on the path, the compiler's wait
        // counts turn conservative and a consumer waits for the newest
        // prefetches too.
        const int lo = lane * 16;   // a lane's 16 bytes of a tile
        // 16-byte loads for the key tiles, 4-byte loads for the rest: w, v
        // and the M T slice of this wave's rows only (W o V reaches the other
        // waves through the partial exchange), and the scalar vectors whose
        // entries a row broadcast hands to the lanes.  The key tiles serve
        // the workgroup's CT column tiles.
        auto load_ops = [&](int j, Ops &o) __attribute__((always_inline)) {
            const int sb = (cw0 + j) * (FB * 4);
#pragma unroll
            for (int kt = 0; kt < KPW; ++kt) {
                const int kg = ks * KPW + kt;
                o.e[kt] = BufF4(rblk, lo, sb + (oE + kg * 256) * 4);
                o.r[kt] = BufF4(rblk, lo, sb + (oR + kg * 256) * 4);
            }
            const Rsrc rw = MakeRsrc(w_run + chunk_off(j), rows_bytes(j));
            const Rsrc rv = MakeRsrc(v_run + chunk_off(j), rows_bytes(j));
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    o.w[c][m] = BufF(rw, vl[c][m]);
                    o.v[c][m] = BufF(rv, vl[c][m]);
                }
#pragma unroll
            for (int x = 0; x < NSV; ++x) o.sc[x] = BufF(rblk, so + x * 256, sb + oSc * 4);
#pragma unroll
            for (int m = 0; m < NM; ++m) o.mt[m] = BufF(rblk, mo[m], sb + oMT * 4);
#pragma unroll
            for (int kt = 0; kt < KPW; ++kt) {
                const int kg = ks * KPW + kt;
                o.ut[kt] = BufF4(rblk, lo, sb + (oU + kg * 256) * 4);
            }
        };

        // One chunk: partial E' S0, R' S0 over this wave's keys, summed across
        // the KS waves (one barrier; the partial buffers alternate by chunk
        // parity, so a wave that runs ahead writes the other buffer, and cannot
        // run two chunks ahead past the next barrier); y = WV - km o E' S0;
        // O = qm o R' S0 + (M T) y (wave 0); S = G_15 o S + Ut~^T y (Ut~ holds
        // T and k_mul).  The next chunk's operands are loaded as described below.
        // The output of a chunk, O = q_mul o R' S0 + (M T) Y, as this wave's
        // partial: its keys of R' S0 and its K slices of (M T) Y (the ii of the
        // 4 with ii % KS == ks); published with the next chunk's E' S0 partials
        // and summed row by row across the waves, so the output products and
        // their reduction are spread over the waves.
        // Partial c of wave z, kind x (0: E' S0, 1: output) sits at
        // ((z 2 + x) CT + c) 256 of a parity's buffer.
        v4f op[CT];
#pragma unroll
        for (int c = 0; c < CT; ++c) op[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        auto part = [&](float *xp, int z, int x, int c) { return xp + ((z * 2 + x) * CT + c) * 256 + lane * 4; };
        auto store_out = [&](int c, int jl, const v4f &out) __attribute__((always_inline)) {   // chunk jl of the run
            const Rsrc ro = MakeRsrc(out_run + out_off(jl), out_bytes(jl));
#pragma unroll
            for (int i = 0; i < 4; ++i) BufStF(ro, oo[c][i], out[i]);
        };
        // The output of chunk jl from the waves' partials, added in wave order.
        // kSpreadOut: wave ks sums and stores token rows i = ks + m KS, so that
        // no wave carries the whole reduction between two barriers; else wave
        // 0 sums and stores every row.  Interleaved A/B, spread against wave 0:
        // sequence-split runs 2 x 2048 x 4 heads at 320 x 64 0.1415 -> 0.1391 ms,
        // 1 x 8192 x 4 heads 0.1563 -> 0.1517; two waves per tile 4 x 4096 x 16
        // heads at 64 x 64 0.3092 -> 0.3015; but four waves per tile (unsplit)
        // 4 x 4096 x 16 heads at 128 x 128 0.5113 -> 0.5208, 16k x 8 heads at
        // 256 x 256 1.2884 -> 1.3057, 8 x 2048 x 16 heads 0.4529 -> 0.4663.
        constexpr bool kSpreadOut = SPLIT || KS <= 3;
        auto sum_out = [&](float *xp, int c) __attribute__((always_inline)) -> v4f {   // wave 0's form
            v4f out = LdsF4(part(xp, 0, 1, c));
#pragma unroll
            for (int z = 1; z < KS; ++z) out += LdsF4(part(xp, z, 1, c));
            return out;
        };
        auto sum_store_out = [&](float *xp, int jl) __attribute__((always_inline)) {   // the spread form
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const Rsrc ro = MakeRsrc(out_run + out_off(jl), out_bytes(jl));
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    const int i = min(ks + m * KS, 3);   // rows >= 4: read row 3, store dropped
                    float out = part(xp, 0, 1, c)[i];
#pragma unroll
                    for (int z = 1; z < KS; ++z) out += part(xp, z, 1, c)[i];
                    BufStF(ro, ol[c][m], out);
                }
            }
        };
        // Vector loads issued in a burst queue behind each other (the CU's
        // waves issue them together); placed one after each MFMA of the
        // products before the barrier, their issue overlaps the products.
        // Where the operand loads of the next chunk are issued: at the end of
        // a step, into its own set (chunk j + 2), the loop's back edge sits
        // between them and the products on every second step; at the head of
        // a step, into the other set (chunk j + 1, that set consumed by the
        // previous step), every step interleaves them.  Measured per key
        // tiling (interleaved A/B): head loads for 4 key tiles per wave and
        // for 3 x 8 (16k tokens x 8 heads at 256 x 256 1.52 -> 1.42 ms, 2 x
        // 2048 x 4 heads at 512 x 64 0.336 -> 0.312, at 384 x 64 0.265 ->
        // 0.253), end-of-step loads elsewhere (head loads: 4 x 4096 x 16
        // heads at 64 x 64 0.327 -> 0.344, 2 x 2048 x 4 heads at 320 x 64
        // 0.234 -> 0.244).  With 6 key tiles per wave the interleave measured
        // 2% slower (4 x 2048 x 16 heads at 384 x 128) and is left out.
        constexpr bool kHeadLoads = KPW == 4 || (KPW == 3 && KS == 8);
        constexpr int kLoads = 3 * KPW + NSV + NM + 2 * CT * NM;   // vector loads of one chunk
        auto interleave = [&]() __attribute__((always_inline)) {
            if constexpr (KPW == 6) return;
#pragma unroll
            for (int i = 0; i < kLoads; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // one vector-memory read
            }
        };
        auto step = [&](int j, Ops &o, Ops &nx) __attribute__((always_inline)) {
            v4f xe[CT], xr[CT];
#pragma unroll
            for (int c = 0; c < CT; ++c) xe[c] = xr[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kt = 0; kt < KPW; ++kt) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
#pragma unroll
                    for (int c = 0; c < CT; ++c) {
                        xe[c] = Mfma(o.e[kt][ii], S[c][kt][ii], xe[c]);
                        xr[c] = Mfma(o.r[kt][ii], S[c][kt][ii], xr[c]);
                    }
                }
            }
            if constexpr (kHeadLoads) load_ops(min(j + 1, nrun - 1), nx);
            v4f wv[CT];   // W o V of this lane's rows; w, v are zero past the sequence end and dv
            if constexpr (KS > 1) {
                float *const xp = sXp + (j & 1) * L::kPart;
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    StF4(part(xp, ks, 0, c), xe[c]);
                    StF4(part(xp, ks, 1, c), op[c]);   // output partial of chunk j - 1
                }
                float *const xw = xp + KS * 2 * CT * 256;   // W o V [CT][256], then the spare row slot
#pragma unroll
                for (int m = 0; m < NM; ++m) {   // this wave's rows of W o V (rows >= 4: the spare slot)
                    const int i = ks + m * KS;
#pragma unroll
                    for (int c = 0; c < CT; ++c) xw[i < 4 ? c * 256 + lane * 4 + i : CT * 256 + lane] = o.w[c][m] * o.v[c][m];
                }
                interleave();
                __syncthreads();
                // the same summation order in every wave: identical Y everywhere
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    xe[c] = LdsF4(part(xp, 0, 0, c));
#pragma unroll
                    for (int z = 1; z < KS; ++z) xe[c] += LdsF4(part(xp, z, 0, c));
                    wv[c] = LdsF4(xw + c * 256 + lane * 4);
                }
                if constexpr (kSpreadOut) {
                    if (j > 0) sum_store_out(xp, j - 1);
                } else if (ks == 0 && j > 0) {
#pragma unroll
                    for (int c = 0; c < CT; ++c) store_out(c, j - 1, sum_out(xp, c));
                }
            } else {
#pragma unroll
                for (int c = 0; c < CT; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) wv[c][i] = o.w[c][i] * o.v[c][i];   // NM = 4: row m is row i
            }
            v4f y[CT];
            const v4f km = KMulRows(o.sc);
#pragma unroll
            for (int c = 0; c < CT; ++c) y[c] = wv[c] - km * xe[c];   // rows of E' S0 times k_mul
            // S = G_15 o S + Ut~^T Y (Ut~ carries T and k_mul: U is never formed)
#pragma unroll
            for (int c = 0; c < CT; ++c) DecayState(S[c], o.sc, std::make_integer_sequence<int, KPW>{});
#pragma unroll
            for (int kt = 0; kt < KPW; ++kt) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
#pragma unroll
                    for (int c = 0; c < CT; ++c) S[c][kt] = Mfma(o.ut[kt][ii], y[c][ii], S[c][kt]);
                }
            }
            // Off the chunk's chain (U, then the update): this wave's K slices
            // of (M T) Y, chosen by selects rather than branches (a branch per
            // slice split the region and delayed U behind them).
            const v4f qm = QMulRows(o.sc);
#pragma unroll
            for (int c = 0; c < CT; ++c) op[c] = qm * xr[c];   // rows of R' S0 times q_mul
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const int sel = ks + m * KS;   // wave-uniform; >= 4 for the waves without a slice
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    float ya = 0.0f;
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) ya = sel == ii ? y[c][ii] : ya;
                    if (m * KS < 4) op[c] = Mfma(sel < 4 ? o.mt[m] : 0.0f, ya, op[c]);
                }
            }
            if constexpr (KS == 1) {
#pragma unroll
                for (int c = 0; c < CT; ++c) store_out(c, j, op[c]);
            }
            if constexpr (!kHeadLoads) load_ops(min(j + 2, nrun - 1), o);
        };

        // two operand sets in turn, with compile-time roles
        // (the sets' loads in the same order as in the loop: an interleaved
        // prologue would set the loop's wait counts to its own, shorter distances)
        Ops opa, opb;
        load_ops(0, opa);
        if constexpr (!kHeadLoads) {
            __builtin_amdgcn_sched_barrier(0);
            load_ops(min(1, nrun - 1), opb);
        }
        // each step leaves the loop or goes on to the other set's step: a path
        // from one set's step back to itself (no newer loads outstanding, to the
        // compiler) would take its wait counts to zero
        for (int j = 0;; j += 2) {
            step(j, opa, opb);
            if (j + 1 >= nrun) break;
            step(j + 1, opb, opa);
            if (j + 2 >= nrun) break;
        }
        if constexpr (KS > 1) {   // output of the last chunk
            float *const xp = sXp + (nrun & 1) * L::kPart;
#pragma unroll
            for (int c = 0; c < CT; ++c) StF4(part(xp, ks, 1, c), op[c]);
            __syncthreads();
            if constexpr (kSpreadOut) {
                sum_store_out(xp, nrun - 1);
            } else if (ks == 0) {
#pragma unroll
                for (int c = 0; c < CT; ++c) store_out(c, nrun - 1, sum_out(xp, c));
            }
            __syncthreads();   // the partial buffers are reused by the workgroup's next run
        }
    }
    if (s_out != nullptr) {
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            const int oc = ocol[c];
            if (!ocol_ok[c]) continue;
#pragma unroll
            for (int kt = 0; kt < KPW; ++kt) {
                const int kb = (ks * KPW + kt) * 16 + 4 * g4;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (kb + i < dk) s_out[sbase + static_cast<size_t>(kb + i) * OW + oc] = S[c][kt][i];
            }
        }
    }
}

// Unpacked: a workgroup owns (b, h, column tile) and the window's wn chunks
// of its sequence, the state from s_in to s_out.
// Packed (chunk_off set): the window holds chunks [c0, c0 + W) of every
// sequence, sequence b's at blocks [chunk_off[b], chunk_off[b + 1]) of each
// head's wn blocks.  Workgroup (slot, h, column tile) takes sequences slot,
// slot + slots, ... that have chunks in the window.  A range that starts the
// sequence reads initial_state (zeros when absent), any other the carry
// (p.state); one that ends it writes final_state (if requested), any other
// the carry, in place: a workgroup reads and writes only its own rows and
// columns.
template <int KPW, int KS, int CT, bool PACKED>
__global__ __launch_bounds__(64 * KS) void Gdn2ChunkRecurKernel(GatedDeltaNet2Params p, int c0, int wn,
                                                                const float *s_in, float *s_out) {
    using L = RecurLayout<KPW, KS, CT>;
    __shared__ __attribute__((aligned(16))) float sXp[L::kFloats];
    const int H = p.nheads;
    const int VW = ((p.dv + 15) / 16 + CT - 1) / CT;   // workgroups per (b, h)
    const int row = XcdLocalBlock(blockIdx.x, gridDim.x) / VW;
    const size_t kv = static_cast<size_t>(p.dk) * p.dv;
    if constexpr (!PACKED) {
        const int b = row / H, h = row % H;
        Gdn2RecurRun<KPW, KS, CT>(p, sXp, h, static_cast<size_t>(b) * p.seqlen, p.seqlen, c0, 0, wn, wn,
                                  p.prepared + static_cast<size_t>(row) * wn * L::FB, static_cast<size_t>(row) * kv,
                                  s_in, s_out);
        return;
    } else {
    const int n = p.batch;
    const int slots = static_cast<int>(gridDim.x) / (H * VW);
    const int slot = row / H, h = row % H;
    const float *const prep_row = p.prepared + static_cast<size_t>(h) * wn * L::FB;
    for (int b = slot; b < n; b += slots) {   // workgroup-uniform
        const int i0 = p.chunk_off[b], nrun = p.chunk_off[b + 1] - i0;
        if (nrun <= 0) continue;   // no chunks in this window
        size_t tok0;
        int T;
        PackedRange(p, b, tok0, T);
        const int nch = (T + kC - 1) / kC;
        const size_t sbase = (static_cast<size_t>(b) * H + h) * kv;
        const float *in = c0 == 0 ? p.initial_state : p.state;
        float *out = c0 + nrun == nch ? p.final_state : p.state;
        Gdn2RecurRun<KPW, KS, CT>(p, sXp, h, tok0, T, c0, i0, nrun, wn, prep_row, sbase, in, out);
    }
    }
}

// ---------------------------------------------------------------------------
// Sequence split (launches with few column-tile workgroups)
// ---------------------------------------------------------------------------
// The state after a run of chunks is affine in the state before it:
// S_end = Phi S_start + S0 (S0: the run from a zero state), and so are its
// outputs: O = O0 + Psi S_start.  The chunks are cut into nseg segments of sc;
// all segments run at once, segment 0 from the initial state and the others
// from zero, the latter with dk identity columns beside the value columns (WV
// = 0, state I), whose outputs are Psi and whose final state is Phi.  The
// combine kernel then steps S_start(s + 1) = Phi_s S_start(s) + S0_s over the
// segments, and the correction kernel adds Psi_s S_start(s) to their outputs.
//
// Workgroup ((b, h), segment, column tile): segment 0 runs its VT value tiles,
// the others VT + KT tiles, VT + (nseg - 1)(VT + KT) workgroups per (b, h) in
// that order.  Each XCD owns a contiguous range of these logical indices
// (XcdLocalBlock), so the XCDs get equal shares of the launch and the
// workgroups of one (b, h), which read the same prepared blocks, share an L2.
// (Ordered by segment first, the later segments' workgroups crowded onto some
// XCDs, two to a CU, while segment 0's left others idle.)  Value tiles write
// O0 (O for segment 0) and S0_s ([nseg][B*H][K][V]); identity tiles write Psi
// ([B,T,H,K], tokens of segments >= 1) and Phi_s ([nseg][B*H][K][K], row =
// key, column = identity column).
template <int KPW, int KS>
__global__ __launch_bounds__(64 * KS) void Gdn2ChunkSplitKernel(GatedDeltaNet2Params p, int sc, int nchunks,
                                                                float *psi, float *phi, float *s0) {
    using L = RecurLayout<KPW, KS, 1>;
    __shared__ __attribute__((aligned(16))) float sXp[L::kFloats];
    const int H = p.nheads, VT = (p.dv + 15) / 16, KT = (p.dk + 15) / 16, tiles = VT + KT;
    const int rows = p.batch * H;
    const int nseg = (nchunks + sc - 1) / sc;
    const int per_row = VT + (nseg - 1) * tiles;
    const int x = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int row = x / per_row, rx = x % per_row;
    const int seg = rx < VT ? 0 : 1 + (rx - VT) / tiles;
    const int tile = rx < VT ? rx : (rx - VT) % tiles;
    const int cs = seg * sc, nrun = min(sc, nchunks - cs);
    if (nrun <= 0) return;
    const int b = row / H, h = row % H;
    const bool ident = tile >= VT;
    const size_t kv = static_cast<size_t>(p.dk) * p.dv, kp = static_cast<size_t>(p.dk) * KT * 16;
    const float *s_in = seg == 0 && p.initial_state != nullptr ? p.initial_state + row * kv : nullptr;
    float *s_out = ident ? phi + (static_cast<size_t>(seg) * rows + row) * kp : s0 + (static_cast<size_t>(seg) * rows + row) * kv;
    Gdn2RecurRun<KPW, KS, 1, true>(p, sXp, h, static_cast<size_t>(b) * p.seqlen, p.seqlen, cs, cs, nrun, nchunks,
                                p.prepared + static_cast<size_t>(row) * nchunks * L::FB, 0, s_in, s_out,
                                SplitTile{tile, ident, psi});
}

// Two unequal segments for launches whose value tiles fill at most half the
// CUs and whose identity tiles are too many for one more workgroup per CU at
// one tile each (e.g. 1 x 8 heads at 256 x 256: 128 value tiles, 256 value and
// key tiles in a second segment).  Segment 0, chunks [0, sc), runs its VT value
// tiles one per workgroup; segment 1, chunks [sc, nchunks), runs its value and
// identity tiles two per workgroup (ceil(VT / 2) + ceil(KT / 2) workgroups),
// which steps a chunk in about 1.6 times segment 0's time when both run.  So
// segment 0 is the longer one, and the launch has one workgroup per CU for
// both.  Workgroups per (b, h): segment 0's tiles, then segment 1's pairs;
// outputs as in Gdn2ChunkSplitKernel with nseg = 2.
template <int KPW, int KS>
__global__ __launch_bounds__(64 * KS) void Gdn2ChunkSplit2Kernel(GatedDeltaNet2Params p, int sc, int nchunks,
                                                                 float *psi, float *phi, float *s0) {
    using L1 = RecurLayout<KPW, KS, 1>;
    using L2 = RecurLayout<KPW, KS, 2>;
    static_assert(L1::FB == L2::FB && L1::kFloats <= L2::kFloats, "one block layout, the two-tile partials");
    __shared__ __attribute__((aligned(16))) float sXp[L2::kFloats];
    const int H = p.nheads, VT = (p.dv + 15) / 16, KT = (p.dk + 15) / 16;
    const int VP = (VT + 1) / 2, per_row = VT + VP + (KT + 1) / 2;
    const int rows = p.batch * H;
    const int x = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int row = x / per_row, rx = x % per_row;
    const int b = row / H, h = row % H;
    const size_t kv = static_cast<size_t>(p.dk) * p.dv, kp = static_cast<size_t>(p.dk) * KT * 16;
    const float *const prep_row = p.prepared + static_cast<size_t>(row) * nchunks * L1::FB;
    const size_t tok0 = static_cast<size_t>(b) * p.seqlen;
    if (rx < VT) {   // workgroup-uniform
        const float *s_in = p.initial_state != nullptr ? p.initial_state + row * kv : nullptr;
        Gdn2RecurRun<KPW, KS, 1, true>(p, sXp, h, tok0, p.seqlen, 0, 0, min(sc, nchunks), nchunks, prep_row, 0, s_in,
                                       s0 + static_cast<size_t>(row) * kv, SplitTile{rx, false, psi});
    } else {
        const int nrun = nchunks - sc;
        if (nrun <= 0) return;
        const int u = rx - VT;
        const bool ident = u >= VP;
        float *s_out = ident ? phi + (static_cast<size_t>(rows) + row) * kp : s0 + (static_cast<size_t>(rows) + row) * kv;
        Gdn2RecurRun<KPW, KS, 2, true>(p, sXp, h, tok0, p.seqlen, sc, sc, nrun, nchunks, prep_row, 0, nullptr, s_out,
                                       SplitTile{u, ident, psi});
    }
}

// Stages column tile vt of a [dk][dv] state (row base src, workgroup-uniform)
// in LDS column by column at pitch SP, keys padded to 16 KT with zeros: NT
// threads, each with B loads in flight before their LDS writes (one load,
// wait and write per element serialises the loads' latency: 20 of them at
// 320 keys).  Byte offsets are 32-bit (a state row is under 2 GiB), so each
// load takes one offset register beside the uniform base.
template <int NT, int B>
__device__ __forceinline__ void StageStateTile(float *dst, const float *src, int dk, int dv, int vt, int KT, int SP,
                                               int tid) {
    const int n = KT * 256, c = vt * 16 + tid % 16;
    const char *const base = reinterpret_cast<const char *>(src);
    for (int i0 = 0; i0 < n; i0 += B * NT) {
        float v[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int i = i0 + u * NT + tid, key = i / 16;
            const unsigned off = static_cast<unsigned>(key * dv + c) * 4u;
            v[u] = i < n && key < dk && c < dv ? *reinterpret_cast<const float *>(base + off) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int i = i0 + u * NT + tid;
            if (i < n) dst[(tid % 16) * SP + i / 16] = v[u];
        }
    }
}

// Workgroup ((b, h), value tile), 8 waves: S (keys x 16 columns, keys padded
// to 16) in LDS, S_start(1) = S0_0; for s >= 1 it stores S_start(s) to sst and
// forms S_start(s + 1) = Phi_s S_start(s) + S0_s on MFMA, wave w taking the
// 16-key output tiles w, w + 8, ...; the last one is the final state, formed
// only when it is requested.  Phi rows
// (pitch KP, 16-byte aligned) are read 16 bytes a lane.  A wave's first tile
// has its first eight key tiles of Phi_{s+1} and its S0_{s+1} values loaded
// during step s (the steps are serial: each would otherwise wait out its
// loads); further key tiles are loaded eight at a time.  S is stored column
// by column (pitch KP + 4 floats: the 16 columns' rows fall in different
// banks), so a lane reads its four B-operand keys with one 16-byte LDS read.
// Dynamic LDS: two buffers of 16 (KP + 4) floats.
__global__ __launch_bounds__(512) void Gdn2SplitCombineKernel(GatedDeltaNet2Params p, int nseg, const float *phi,
                                                               const float *s0, float *sst) {
    extern __shared__ float comb[];
    const int dk = p.dk, dv = p.dv, VT = (dv + 15) / 16, KT = (dk + 15) / 16, KP = KT * 16;
    const int rows = p.batch * p.nheads;
    const int row = blockIdx.x / VT, vt = blockIdx.x % VT;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, m16 = lane & 15, g4 = lane >> 4;
    const size_t kv = static_cast<size_t>(dk) * dv, kp = static_cast<size_t>(dk) * KP;
    const int col = vt * 16 + m16;
    const int SP = KP + 4;   // LDS pitch of one column of S
    float *cur = comb, *nxt = comb + 16 * SP;
    StageStateTile<512, 8>(cur, s0 + row * kv, dk, dv, vt, KT, SP, tid);
    // A[m][k] = Phi_s[16 kt + m][k] (lane m + 16 k, 16 bytes per key tile);
    // S0_s at the D layout (key 16 kt + 4 (l / 16) + i, column l % 16)
    auto load_a = [&](int s, int kt, int k0, v4f (&a)[8]) __attribute__((always_inline)) {
        const int arow = kt * 16 + m16;
        const float *const prow = phi + (static_cast<size_t>(s) * rows + row) * kp +
                                  static_cast<size_t>(arow < dk ? arow : 0) * KP + 4 * g4;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
            a[u] = arow < dk && k0 + u < KT ? *reinterpret_cast<const v4f *>(prow + (k0 + u) * 16) : z;
        }
    };
    auto load_add = [&](int s, int kt) __attribute__((always_inline)) -> v4f {
        const float *const add = s0 + (static_cast<size_t>(s) * rows + row) * kv;
        v4f r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = kt * 16 + 4 * g4 + i;
            r[i] = key < dk && col < dv ? add[static_cast<size_t>(key) * dv + col] : 0.0f;
        }
        return r;
    };
    auto products = [&](v4f acc, const v4f (&a)[8], int k0) __attribute__((always_inline)) -> v4f {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (k0 + u >= KT) break;
            const v4f bs = LdsF4(cur + m16 * SP + (k0 + u) * 16 + 4 * g4);   // B[k][n] = S[16 kb + 4 k + ii][n]
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) acc = Mfma(a[u][ii], bs[ii], acc);
        }
        return acc;
    };
    const bool first = w < KT;   // this wave's first tile, kt = w
    // the products of step s form S_start(s + 1): the last one only for the final state
    const int nprod = p.final_state != nullptr ? nseg : nseg - 1;
    v4f a0[8], a1[8], add0 = {0.0f, 0.0f, 0.0f, 0.0f}, add1 = add0;
    if (first && nprod > 1) {
        load_a(1, w, 0, a0);
        add0 = load_add(1, w);
    }
    __syncthreads();
    for (int s = 1; s < nseg; ++s) {   // workgroup-uniform
        float *const start = sst + (static_cast<size_t>(s) * rows + row) * kv;
        for (int i = tid; i < KT * 256; i += 512) {
            const int key = i / 16, c = vt * 16 + i % 16;
            if (key < dk && c < dv) start[static_cast<size_t>(key) * dv + c] = cur[(i % 16) * SP + key];
        }
        if (s >= nprod) break;   // workgroup-uniform: no final state wanted
        if (first) {
            if (s + 1 < nprod) {   // the next step's operands, in flight during this one
                load_a(s + 1, w, 0, a1);
                add1 = load_add(s + 1, w);
            }
            v4f acc = products(add0, a0, 0);
            for (int k0 = 8; k0 < KT; k0 += 8) {
                v4f a[8];
                load_a(s, w, k0, a);
                acc = products(acc, a, k0);
            }
            StF4(nxt + m16 * SP + w * 16 + 4 * g4, acc);
#pragma unroll
            for (int u = 0; u < 8; ++u) a0[u] = a1[u];
            add0 = add1;
        }
        for (int kt = w + 8; kt < KT; kt += 8) {   // keys beyond 128: further tiles
            v4f acc = load_add(s, kt);
            for (int k0 = 0; k0 < KT; k0 += 8) {
                v4f a[8];
                load_a(s, kt, k0, a);
                acc = products(acc, a, k0);
            }
            StF4(nxt + m16 * SP + kt * 16 + 4 * g4, acc);
        }
        __syncthreads();
        float *const t = cur;
        cur = nxt;
        nxt = t;
    }
    if (p.final_state != nullptr) {
        float *const fs = p.final_state + row * kv;
        for (int i = tid; i < KT * 256; i += 512) {
            const int key = i / 16, c = vt * 16 + i % 16;
            if (key < dk && c < dv) fs[static_cast<size_t>(key) * dv + c] = cur[(i % 16) * SP + key];
        }
    }
}

// O += Psi_s S_start(s) over the tokens of segment s >= 1 (chunks [s sc,
// min((s + 1) sc, nchunks))): workgroup ((b, h), value tile, s, four
// consecutive chunks of the segment; ncg such groups per segment), a wave per
// chunk, S_start(s)'s column tile staged in LDS.  D[m][n] = sum_k Psi[t0 + m][k]
// S_start[k][n] on MFMA (A: lane m + 16 k holds Psi[t0 + m][16 kb + 4 k + ii],
// 16 bytes of a KP-pitch row; B from LDS, stored column by column at pitch
// KP + 4 for 16-byte reads), added to the output rows.  Dynamic LDS:
// 16 (KP + 4) floats.
// s1 (or null): segment 1's start state at the row's [K][V] of s1, in place
// of sst (a split in two segments with no final state has no combine step:
// segment 0's final state is segment 1's start).
// SB: state loads in flight per thread while staging.  16 takes the kernel
// from 50 to 112 VGPRs (4 waves per SIMD instead of 8): worth it only where
// every workgroup is resident at once and each waits out its own staging.
template <int SB>
__global__ __launch_bounds__(256) void Gdn2SplitCorrectKernel(GatedDeltaNet2Params p, int sc, int ncg, int nchunks,
                                                              const float *psi, const float *sst, const float *s1) {
    extern __shared__ float sts[];
    const int dk = p.dk, dv = p.dv, H = p.nheads, T = p.seqlen, VT = (dv + 15) / 16, KT = (dk + 15) / 16;
    const int KP = KT * 16, rows = p.batch * H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, m16 = lane & 15, g4 = lane >> 4;
    // value tile fastest, each XCD a contiguous range: the VT workgroups of
    // one group of chunks run together on one XCD and read its Psi rows
    // through one L2 (ordered chunk group first, a Psi row was fetched once per
    // value tile: 1 x 16384 x 8 heads at 256 x 256 with the two-tile split,
    // 1.188 -> 1.171 ms, interleaved A/B)
    const int x = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int vt = x % VT, cg = (x / VT) % ncg, row = (x / VT / ncg) % rows, seg = 1 + x / VT / ncg / rows;
    const int b = row / H, h = row % H;
    const int c = seg * sc + cg * 4 + w;
    const bool live = cg * 4 + w < sc && c < nchunks;   // whole wave
    const int col = vt * 16 + m16;
    const int ta = c * kC + m16;   // this lane's A-operand token
    const bool ta_ok = live && ta < T;
    const float *const prow = psi + ((static_cast<size_t>(b) * T + (ta_ok ? ta : 0)) * H + h) * KP + 4 * g4;
    v4f a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {   // the first eight key tiles' loads before the staging wait
        const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
        a[u] = ta_ok && u < KT ? *reinterpret_cast<const v4f *>(prow + u * 16) : z;
    }
    float *const orow = p.out + ((static_cast<size_t>(b) * T + c * kC + 4 * g4) * H + h) * dv + col;
    float o[4];   // the output values the products add to, loaded with the first operands
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = c * kC + 4 * g4 + i;
        o[i] = live && t < T && col < dv ? orow[static_cast<size_t>(i) * H * dv] : 0.0f;
    }
    const size_t kv = static_cast<size_t>(dk) * dv;
    const float *const st = seg == 1 && s1 != nullptr ? s1 + static_cast<size_t>(row) * kv
                                                      : sst + (static_cast<size_t>(seg) * rows + row) * kv;
    const int SP = KP + 4;
    StageStateTile<256, SB>(sts, st, dk, dv, vt, KT, SP, tid);
    __syncthreads();
    if (!live) return;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < KT; k0 += 8) {
        if (k0 > 0) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
                a[u] = ta_ok && k0 + u < KT ? *reinterpret_cast<const v4f *>(prow + (k0 + u) * 16) : z;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (k0 + u >= KT) break;
            const v4f bs = LdsF4(sts + m16 * SP + (k0 + u) * 16 + 4 * g4);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) acc = Mfma(a[u][ii], bs[ii], acc);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = c * kC + 4 * g4 + i;
        if (t < T && col < dv) orow[static_cast<size_t>(i) * H * dv] = o[i] + acc[i];
    }
}

// O += Psi S_start(s) over the chunks [s sc, min((s + 1) sc, nchunks)) of
// every segment s >= 1, with KTM >= ceil(dk / 16) key tiles: workgroup (s,
// (b, h), block of cpw chunks of the segment, group of four value tiles),
// value-tile group fastest (in XCD-local order the groups of one chunk block
// run together and read its Psi rows through one L2); ncb blocks per segment.
// S_start(s) is at sst's [s][B*H][K][V], or for s = 1 at s1 when given (two
// segments with no final state: segment 0's final state is segment 1's
// start).  Wave w holds value tile 4 g + w of S_start(s) in VGPRs as MFMA B
// operands (lane l: keys 16 kt + 4 (l / 16) + ii, column l % 16).  Per chunk the workgroup stages the chunk's Psi tile (16
// token rows of KP keys) in LDS once, and each wave multiplies it by its
// state tile: D[m][n] = sum_k Psi[t0 + m][k] S_start[k][n] (A: lane m + 16 k
// reads Psi[t0 + m][16 kt + 4 k + ii]), added to the output rows.  Read from
// L2 by every wave (16 KB per 64 MFMAs), the A operands held the CU's vector
// memory path at its limit: 117 us at 1 x 16384 x 8 heads, 256 x 256.  Psi
// and output rows go through per-chunk raw-buffer descriptors that end after
// the chunk's last valid token (zeros past it; keys past KP read as zeros);
// the next chunk's tile loads into registers while a chunk multiplies, and
// goes to the other of two LDS buffers (one barrier per chunk).  The MFMAs
// alternate over four accumulators.  LDS rows at a pitch of KTM 16 + 8
// floats (8 x odd: row-strided 16-byte reads without bank conflicts).  The
// host keeps H KP and H dv under 2^25 and dk dv under 2^29.
template <int KTM>
__global__ __launch_bounds__(256) void Gdn2SplitCorrectRegKernel(GatedDeltaNet2Params p, int sc, int ncb, int cpw,
                                                                 int nchunks, const float *psi, const float *sst,
                                                                 const float *s1) {
    constexpr int PS = KTM * 16 + 8;   // LDS row pitch (floats)
    constexpr int NV = KTM / 4;        // 16-byte loads per thread per tile
    __shared__ __attribute__((aligned(16))) float sa[2][kC * PS];
    const int dk = p.dk, dv = p.dv, H = p.nheads, T = p.seqlen, VT = (dv + 15) / 16, KT = (dk + 15) / 16;
    const int KP = KT * 16, VG = (VT + 3) / 4, rows = p.batch * H;
    const int tid = threadIdx.x, lane = tid & 63, m16 = lane & 15, g4 = lane >> 4;
    // wave-uniform (readfirstlane): descriptors built from a lane-varying
    // value would put every buffer load in a waterfall loop
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(tid >> 6));
    const long long x = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int vg = static_cast<int>(x % VG);
    const long long rc = x / VG;
    const int cb = static_cast<int>(rc % ncb), row = static_cast<int>(rc / ncb % rows);
    const int seg = 1 + static_cast<int>(rc / ncb / rows);
    const int b = row / H, h = row % H;
    const int col = (4 * vg + wave) * 16 + m16;
    const size_t kv = static_cast<size_t>(dk) * dv;
    const float *const st = (seg == 1 && s1 != nullptr ? s1 : sst + static_cast<size_t>(seg) * rows * kv) + row * kv;
    const bool col_ok = col < dv;   // false in every lane of a wave past the value tiles: zeros, stores dropped
    const Rsrc rs = MakeRsrc(st, dk * dv * 4);
    float S[KTM][4];
#pragma unroll
    for (int kt = 0; kt < KTM; ++kt)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int key = 16 * kt + 4 * g4 + ii;
            S[kt][ii] = BufF(rs, key < dk && col_ok ? (key * dv + col) * 4 : kOutOfRange);
        }
    const int cbeg = seg * sc + cb * cpw, cend = min(min(cbeg + cpw, (seg + 1) * sc), nchunks);   // workgroup-uniform
    const int HKP4 = H * KP * 4, HD4 = H * dv * 4;
    // staging: thread t copies the 16-byte pieces 16 v + t % 16 (v < NV) of
    // token row t / 16, so the 16 threads of a row read 256 contiguous bytes
    // and write them to 64 distinct banks (keys past KP out of range: zeros)
    const int srow = tid >> 4, sseg = (tid & 15) * 4;
    int so[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) so[v] = sseg + 64 * v < KP ? srow * HKP4 + (sseg + 64 * v) * 4 : kOutOfRange;
    int oo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) oo[i] = col_ok ? (4 * g4 + i) * HD4 + col * 4 : kOutOfRange;
    auto rows_rsrc = [&](const float *xr, int w, int c) __attribute__((always_inline)) {   // chunk c's token rows of width w
        c = __builtin_amdgcn_readfirstlane(min(c, nchunks - 1));
        const int left = min(T - c * kC, kC);
        return MakeRsrc(xr + ((static_cast<size_t>(b) * T + c * kC) * H + h) * w, ((left - 1) * H * w + w) * 4);
    };
    v4f pre[NV];
    auto gload = [&](int c) __attribute__((always_inline)) {   // chunk c's Psi tile (clamped to the last chunk)
        const Rsrc rp = rows_rsrc(psi, KP, c);
#pragma unroll
        for (int v = 0; v < NV; ++v) pre[v] = BufF4(rp, so[v], 0);
    };
    auto lstore = [&](float *buf) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < NV; ++v) StF4(buf + srow * PS + sseg + 64 * v, pre[v]);
    };
    auto oload = [&](int c, float (&o)[4]) __attribute__((always_inline)) {
        const Rsrc ro = rows_rsrc(p.out, dv, c);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = BufF(ro, oo[i]);
    };
    gload(cbeg);
    lstore(sa[0]);
    float o[4];
    oload(cbeg, o);
    __syncthreads();
    for (int c = cbeg; c < cend; ++c) {
        float *const cur = sa[(c - cbeg) & 1];
        gload(c + 1);
        float on[4];
        oload(c + 1, on);
        v4f acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kt = 0; kt < KTM; ++kt) {
            const v4f a = LdsF4(cur + m16 * PS + 16 * kt + 4 * g4);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) acc[ii] = Mfma(a[ii], S[kt][ii], acc[ii]);
        }
        const v4f d = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        const Rsrc ro = rows_rsrc(p.out, dv, c);
#pragma unroll
        for (int i = 0; i < 4; ++i) BufStF(ro, oo[i], o[i] + d[i]);
        // the other buffer was last read in iteration c - 1, before its barrier
        lstore(sa[((c - cbeg) & 1) ^ 1]);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = on[i];
    }
}

struct ChunkConfig {
    int kpw, ks;
    int ct = 1;   // value-column tiles per recurrence workgroup
};

// Up to 128 keys: two key tiles (32 keys) per wave, ks = ceil(tiles / 2)
// waves per column tile (keys padded to 32 ks; 3 waves rather than 4 for
// 65-96 keys measured 11-12% faster).  Fewer splits leave too few
// waves for the chip (one wave per SIMD at best, and half the SIMDs idle for
// 4 x 16 heads of 128 x 128): four tiles per wave measured 7-28% slower
// there.  Above 128 keys, three to six key tiles per wave (two tiles per
// wave with 10-16 waves spill), measured 11-22% faster than two tiles per
// wave for 160-256 keys.  A CU has 4 SIMDs, so 5-7 waves put two on some
// SIMD, whose doubled MFMA work every chunk's barrier waits for: 129-192
// keys take 4 waves of 3 tiles (3 waves of 4 before: -2 to -9%); 257-320
// keys 4 waves of 5 tiles (8 waves of 3 or 5 of 4 before: 2 x 2048 x 4
// heads at 288-320 x 64 -11%, 4 x 2048 x 32 heads at 320 x 64 -7%);
// 321-384 keys 8 waves of 3 tiles when the launch has fewer column-tile
// workgroups than half the CUs (4 waves of 6 tiles: +5% at 2 x 2048 x 4
// heads), else 4 waves of 6 tiles (-3% against 6 waves of 4 at 4 x 2048 x
// 16 heads of 384 x 128).  The gdn2_kpw4 override keeps 4 tiles and
// ceil(tiles / 4) waves above 128 keys.  `groups`: the launch's column-tile
// workgroups.
ChunkConfig ChooseKeyTiling(int dk, long long groups) {
    const int kq = (dk + 15) / 16;
    if (kq > 8) {
        if (GetOverride(kOverrideGdn2Kpw4) == 1) return ChunkConfig{4, (kq + 3) / 4};
        if (kq <= 12) return ChunkConfig{3, 4};
        if (kq > 16 && kq <= 20) return ChunkConfig{5, 4};
        if (kq > 20 && kq <= 24) return groups < 128 ? ChunkConfig{3, 8} : ChunkConfig{6, 4};
        return ChunkConfig{4, (kq + 3) / 4};
    }
    ChunkConfig c{kq >= 2 ? 2 : 1, 1};
    const int need = (kq + c.kpw - 1) / c.kpw;
    c.ks = need;
    return c;
}

// Recurrence kernels with two column tiles per workgroup are built for these
// key tilings.
bool HasTwoTileKernel(const ChunkConfig &c) {
    return (c.kpw == 2 && c.ks >= 2 && c.ks <= 4) || (c.kpw == 3 && c.ks == 4) || (c.kpw == 4 && c.ks == 4);
}

// CUs of the current device (cached per device).
int DeviceCus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Two column tiles per workgroup share each key tile's loads and partial
// exchange over twice the MFMA work.  Taken wherever one tile per workgroup
// would put more workgroups than CUs: a CU stepping two workgroups at once
// gains about 14% over one, so the doubled CUs set the kernel's time, and
// half as many two-tile workgroups (one per CU) finish sooner even where some
// CUs then idle (interleaved A/B, 4 x 4096 heads at 128 keys: 16 heads at
// dv = 65 0.545 -> 0.520 ms, at dv = 96 0.554 -> 0.520, at dv = 80 0.542 ->
// 0.534; 12 heads at dv = 128 0.490 -> 0.470).  At or below one workgroup per
// CU halving them idles CUs (16k tokens x 8 heads at 256 x 256: 1.34 -> 2.23
// ms; 4 x 4096 x 16 heads at 64 x 64: 0.33 -> 0.41; 2 x 4096 x 16 heads at
// 128 x 128: 0.325 -> 0.414).
ChunkConfig ChooseChunk(int dk, long long groups) {
    ChunkConfig c = ChooseKeyTiling(dk, groups);
    const int64_t ov = GetOverride(kOverrideGdn2Ct);
    if (HasTwoTileKernel(c) && (ov == 2 || (ov == 0 && groups > DeviceCus()))) c.ct = 2;
    return c;
}

// The preparation kernel, with its Ut' tiles' dynamic LDS (up to 128 KiB at
// 32 key tiles, beside 20 KiB of static LDS).
template <bool AHEAD, int PW>
void LaunchPrepWaves(const ChunkConfig &c, const GatedDeltaNet2Params &p, int c0, int wn, long long items,
                     hipStream_t stream) {
    const long long blocks = (items + PW - 1) / PW;
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    const int dyn = PW * c.kpw * c.ks * 256 * static_cast<int>(sizeof(float));
    EnsureDynamicLds(reinterpret_cast<const void *>(&Gdn2ChunkPrepKernel<AHEAD, PW>), dyn);
    hipLaunchKernelGGL((Gdn2ChunkPrepKernel<AHEAD, PW>), dim3(static_cast<unsigned>(blocks)), dim3(64 * PW), dyn, stream,
                       p, c0, wn, c.kpw, c.ks);
}

void LaunchPrep(const ChunkConfig &c, const GatedDeltaNet2Params &p, int c0, int wn, long long items,
                hipStream_t stream) {
    const int kq = c.kpw * c.ks;
    if (kq > kMaxKeyTiles) throw Error(XM_ERR_DEVICE, "GatedDeltaNet2Fn chunk configuration mismatch");
    // Loads one pair ahead where the Ut' stash in LDS already limits the CU to
    // at most three workgroups (kq > 4); at up to 64 keys the extra registers
    // would take it from four to three.
    const bool ahead = kq > 4 && p.vec4_keys;
    // Above 128 keys the Ut' stash (kq KiB per wave) holds a four-wave
    // workgroup to one per CU; two-wave workgroups fit three per CU (256
    // keys: 6 waves per CU against 4).  Only for launches of 16+ chunk-heads
    // per CU: with fewer, up to three land on some CUs and leave others
    // short.  Interleaved A/B: 1 x 16384 x 8 heads at 256 x 256 (8192 chunk-
    // heads) 1.189 -> 1.166 ms; 2 x 2048 x 4 heads at 320 x 64 (1024) 0.1383 ->
    // 0.1440 with two waves; at 128 keys 0.517 -> 0.519 (VGPRs already bound
    // occupancy there).
    const bool two = kq > 8 && items >= 16LL * DeviceCus();
    if (ahead) {
        if (two) LaunchPrepWaves<true, 2>(c, p, c0, wn, items, stream);
        else LaunchPrepWaves<true, kPrepWaves>(c, p, c0, wn, items, stream);
    } else {
        if (two) LaunchPrepWaves<false, 2>(c, p, c0, wn, items, stream);
        else LaunchPrepWaves<false, kPrepWaves>(c, p, c0, wn, items, stream);
    }
}

template <int KPW, int KS, int CT>
void LaunchRecur(const GatedDeltaNet2Params &p, int c0, int wn, int kq, const float *s_in, float *s_out,
                 hipStream_t stream) {
    if (kq != RecurLayout<KPW, KS, CT>::KQ) throw Error(XM_ERR_DEVICE, "GatedDeltaNet2Fn chunk configuration mismatch");
    const int vt = ((p.dv + 15) / 16 + CT - 1) / CT;   // workgroups per (b, h)
    // packed: min(sequences, chunks) slots per (h, column tile); a slot's
    // workgroup takes every slots-th sequence that meets the window
    const long long rows = p.chunk_off != nullptr ? std::min(p.batch, wn) : p.batch;
    const long long blocks = rows * p.nheads * vt;
    if (blocks == 0) return;   // no packed sequences
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    if (p.chunk_off != nullptr) {
        XM_NOTE_LAUNCH("Gdn2ChunkRecurKernel", {}, KPW, KS, CT, 1);
        hipLaunchKernelGGL((Gdn2ChunkRecurKernel<KPW, KS, CT, true>), dim3(static_cast<unsigned>(blocks)),
                           dim3(64 * KS), 0, stream, p, c0, wn, s_in, s_out);
    } else {
        XM_NOTE_LAUNCH("Gdn2ChunkRecurKernel", {}, KPW, KS, CT, 0);
        hipLaunchKernelGGL((Gdn2ChunkRecurKernel<KPW, KS, CT, false>), dim3(static_cast<unsigned>(blocks)),
                           dim3(64 * KS), 0, stream, p, c0, wn, s_in, s_out);
    }
}

void LaunchRecurAny(const GatedDeltaNet2Params &p, const ChunkConfig &c, int c0, int wn, int kq, const float *s_in,
                    float *s_out, hipStream_t stream) {
#define XM_GDN2_RECUR(KPW_, KS_, CT_)                 \
    if (c.kpw == KPW_ && c.ks == KS_ && c.ct == CT_) \
        return LaunchRecur<KPW_, KS_, CT_>(p, c0, wn, kq, s_in, s_out, stream);
    XM_GDN2_RECUR(1, 1, 1) XM_GDN2_RECUR(2, 1, 1) XM_GDN2_RECUR(2, 2, 1) XM_GDN2_RECUR(2, 3, 1) XM_GDN2_RECUR(2, 4, 1)
    XM_GDN2_RECUR(3, 4, 1) XM_GDN2_RECUR(3, 8, 1) XM_GDN2_RECUR(4, 3, 1) XM_GDN2_RECUR(4, 4, 1) XM_GDN2_RECUR(4, 5, 1)
    XM_GDN2_RECUR(4, 6, 1) XM_GDN2_RECUR(4, 7, 1) XM_GDN2_RECUR(4, 8, 1) XM_GDN2_RECUR(5, 4, 1) XM_GDN2_RECUR(6, 4, 1)
    XM_GDN2_RECUR(2, 2, 2) XM_GDN2_RECUR(2, 3, 2) XM_GDN2_RECUR(2, 4, 2) XM_GDN2_RECUR(3, 4, 2) XM_GDN2_RECUR(4, 4, 2)
#undef XM_GDN2_RECUR
    throw Error(XM_ERR_DEVICE, "GatedDeltaNet2Fn: no chunk kernel for this key tiling");
}

template <int KPW, int KS>
void LaunchSplitRecur(const GatedDeltaNet2Params &p, int nseg, int sc, int nchunks, float *psi, float *phi, float *s0,
                      hipStream_t stream) {
    const long long vt = (p.dv + 15) / 16, tiles = vt + (p.dk + 15) / 16;
    const long long blocks = static_cast<long long>(p.batch) * p.nheads * (vt + (nseg - 1) * tiles);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    XM_NOTE_LAUNCH("Gdn2ChunkSplitKernel", {}, KPW, KS);
    hipLaunchKernelGGL((Gdn2ChunkSplitKernel<KPW, KS>), dim3(static_cast<unsigned>(blocks)), dim3(64 * KS), 0, stream, p,
                       sc, nchunks, psi, phi, s0);
}

template <int KPW, int KS>
void LaunchSplit2Recur(const GatedDeltaNet2Params &p, int sc, int nchunks, float *psi, float *phi, float *s0,
                       hipStream_t stream) {
    const long long vt = (p.dv + 15) / 16, kt = (p.dk + 15) / 16;
    const long long blocks = static_cast<long long>(p.batch) * p.nheads * (vt + (vt + 1) / 2 + (kt + 1) / 2);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    XM_NOTE_LAUNCH("Gdn2ChunkSplit2Kernel", {}, KPW, KS);
    hipLaunchKernelGGL((Gdn2ChunkSplit2Kernel<KPW, KS>), dim3(static_cast<unsigned>(blocks)), dim3(64 * KS), 0, stream,
                       p, sc, nchunks, psi, phi, s0);
}

void LaunchSplitRecurAny(const GatedDeltaNet2Params &p, const ChunkConfig &c, int nseg, int sc, int nchunks, float *psi,
                         float *phi, float *s0, hipStream_t stream) {
#define XM_GDN2_SPLIT(KPW_, KS_) \
    if (c.kpw == KPW_ && c.ks == KS_) return LaunchSplitRecur<KPW_, KS_>(p, nseg, sc, nchunks, psi, phi, s0, stream);
    XM_GDN2_SPLIT(1, 1) XM_GDN2_SPLIT(2, 1) XM_GDN2_SPLIT(2, 2) XM_GDN2_SPLIT(2, 3) XM_GDN2_SPLIT(2, 4)
    XM_GDN2_SPLIT(3, 4) XM_GDN2_SPLIT(3, 8) XM_GDN2_SPLIT(4, 3) XM_GDN2_SPLIT(4, 4) XM_GDN2_SPLIT(4, 5)
    XM_GDN2_SPLIT(4, 6) XM_GDN2_SPLIT(4, 7) XM_GDN2_SPLIT(4, 8) XM_GDN2_SPLIT(5, 4) XM_GDN2_SPLIT(6, 4)
#undef XM_GDN2_SPLIT
    throw Error(XM_ERR_DEVICE, "GatedDeltaNet2Fn: no chunk kernel for this key tiling");
}

void LaunchSplit2RecurAny(const GatedDeltaNet2Params &p, const ChunkConfig &c, int sc, int nchunks, float *psi,
                          float *phi, float *s0, hipStream_t stream) {
#define XM_GDN2_SPLIT2(KPW_, KS_) \
    if (c.kpw == KPW_ && c.ks == KS_) return LaunchSplit2Recur<KPW_, KS_>(p, sc, nchunks, psi, phi, s0, stream);
    XM_GDN2_SPLIT2(2, 2) XM_GDN2_SPLIT2(2, 3) XM_GDN2_SPLIT2(2, 4) XM_GDN2_SPLIT2(3, 4) XM_GDN2_SPLIT2(4, 4)
#undef XM_GDN2_SPLIT2
    throw Error(XM_ERR_DEVICE, "GatedDeltaNet2Fn: no two-tile split kernel for this key tiling");
}

// Sequence split of an unpacked call (see Gdn2ChunkSplitKernel): nseg segments
// of sc chunks, every chunk prepared at once.  Scratch: the prepared blocks
// of every chunk, Psi ([B,T,H,KP]), Phi ([nseg][B*H][K][KP]), S0 and the
// segment start states ([nseg][B*H][K][V] each).  Segments >= 1 run their dk
// identity columns beside the value columns, 1 + dk/dv times the
// recurrence work, in segments of about 64 chunks (at most about 1536
// workgroups beyond segment 0).  A launch of W0 = B*H*VT
// column-tile workgroups (at most one per CU) steps each chunk at the
// latency-bound rate; the split spreads B*H*(VT+KT) tiles' work over the
// CUs at the throughput rate, so it pays when B*H*(VT+KT) is well under the
// CU count: taken at <= 160 and 64+ chunks.  At most 2 GiB of scratch.
struct SplitPlan {
    int nseg = 0, sc = 0, nchunks = 0;
    bool two_tile = false;   // Gdn2ChunkSplit2Kernel: nseg = 2, segment 0 = chunks [0, sc)
    size_t blocks = 0, psi = 0, phi = 0, s0 = 0;
    size_t total() const { return blocks + psi + phi + 2 * s0; }
};

SplitPlan PlanSplit(int batch, int seqlen, int nheads, int dk, int dv, bool packed, size_t cap) {
    const int ov = GetOverride(kOverrideGdn2Split);
    // 128-chunk windows (gdn2_windowed) are the windowed path's test case
    if (packed || ov == 1 || (ov == 0 && GetOverride(kOverrideGdn2Windowed) == 1)) return SplitPlan{};
    const long long rows = static_cast<long long>(batch) * nheads;
    const int VT = (dv + 15) / 16, KT = (dk + 15) / 16;
    const ChunkConfig c = ChooseChunk(dk, rows * VT);
    const int nchunks = (seqlen + kC - 1) / kC;
    const size_t fb = static_cast<size_t>(BlockFloats(c.kpw, c.ks)) * sizeof(float);
    // the recurrence addresses a row's blocks, and 16 tokens of Psi rows, with
    // 32-bit byte offsets
    if (static_cast<size_t>(nchunks) * fb >= (size_t{1} << 31)) return SplitPlan{};
    if (static_cast<long long>(nheads) * KT * 16 >= (1LL << 25)) return SplitPlan{};
    int nseg;
    bool two_tile = false;
    if (ov == 2) {
        nseg = std::min(nchunks, 4);
    } else if (ov == 3) {
        if (!HasTwoTileKernel(c) || nchunks < 2) return SplitPlan{};
        nseg = 2;
        two_tile = true;
    } else if (rows * (VT + KT) > 160) {
        // Wide keys over few value columns (e.g. 2 x 4 heads at 320 x 64: 32
        // column-tile workgroups, 192 value and key tiles): two segments when
        // both fit on the CUs one workgroup each, so the second segment's
        // identity columns run on CUs the unsplit launch leaves idle and
        // every CU still steps at most one workgroup.
        if (nchunks < 64) return SplitPlan{};
        if (rows * VT <= 64 && rows * VT + rows * (VT + KT) <= 256) {
            nseg = 2;
        } else if (HasTwoTileKernel(c) && rows * (VT + (VT + 1) / 2 + (KT + 1) / 2) <= DeviceCus()) {
            // Too many tiles for that, but segment 1 at two tiles per
            // workgroup still fits beside segment 0 (e.g. 1 x 8 heads at
            // 256 x 256: 128 + 128 workgroups): Gdn2ChunkSplit2Kernel.
            nseg = 2;
            two_tile = true;
        } else {
            return SplitPlan{};
        }
    } else {
        if (nchunks < 64) return SplitPlan{};
        // segments of about 64 chunks (longer ones leave the recurrence
        // latency-bound, shorter ones add serial combine steps), at most about
        // 1536 workgroups beyond segment 0.  Measured at 1 x 8192 x 4 heads
        // (128 x 128), 1 x 16384 x 16 heads (64 x 64) and 1 x 8192 x 8 heads
        // (160 x 64), the best of 384 / 768 / 1536 workgroups were 74, 79
        // and 64 chunks per segment.
        const long long per = rows * (VT + KT);
        nseg = std::min((nchunks + 63) / 64, 1 + static_cast<int>((1536 + per - 1) / per));
        nseg = std::max(nseg, 2);
    }
    if (nseg < 2) return SplitPlan{};
    SplitPlan sp;
    if (two_tile) {
        // Segment 0 takes 8 / 13 of the chunks (lengths 1.6 : 1).  Run side
        // by side, a two-tile segment-1 step measured about 1.6 times a
        // one-tile segment-0 step (2.1 against 1.3 us at 1 x 16384 x 8 heads,
        // 256 x 256; each alone: 1.97 against 1.05).  Interleaved A/B of the
        // segment-0 share there: 1.5 : 1 1.184 ms, 1.6 : 1 1.151, 1.7 : 1
        // 1.162, 2.0 : 1 1.213.
        sp.two_tile = true;
        sp.nseg = 2;
        sp.sc = std::min(nchunks - 1, std::max(1, static_cast<int>((static_cast<long long>(nchunks) * 8 + 6) / 13)));
    } else {
        sp.sc = (nchunks + nseg - 1) / nseg;
        sp.nseg = (nchunks + sp.sc - 1) / sp.sc;
    }
    if (sp.nseg < 2) return SplitPlan{};
    sp.nchunks = nchunks;
    sp.blocks = Align256(static_cast<size_t>(rows) * nchunks * fb);
    sp.psi = Align256(static_cast<size_t>(batch) * seqlen * nheads * KT * 16 * sizeof(float));
    sp.phi = Align256(static_cast<size_t>(sp.nseg) * rows * dk * KT * 16 * sizeof(float));
    sp.s0 = Align256(static_cast<size_t>(sp.nseg) * rows * dk * dv * sizeof(float));
    if (sp.total() > std::min(cap, size_t{2} << 30)) return SplitPlan{};
    return sp;
}

void LaunchSplit(const GatedDeltaNet2Params &p, const ChunkConfig &c, const SplitPlan &sp, char *base,
                 hipStream_t stream) {
    GatedDeltaNet2Params q = p;
    q.prepared = reinterpret_cast<float *>(base);
    float *const psi = reinterpret_cast<float *>(base + sp.blocks);
    float *const phi = reinterpret_cast<float *>(base + sp.blocks + sp.psi);
    float *const s0 = reinterpret_cast<float *>(base + sp.blocks + sp.psi + sp.phi);
    float *const sst = reinterpret_cast<float *>(base + sp.blocks + sp.psi + sp.phi + sp.s0);
    const long long rows = static_cast<long long>(p.batch) * p.nheads;
    const int VT = (p.dv + 15) / 16, KT = (p.dk + 15) / 16;
    XM_NOTE_LAUNCH("Gdn2ChunkPrepKernel", {}, );
    LaunchPrep(c, q, 0, sp.nchunks, rows * sp.nchunks, stream);
    XM_LAUNCH_CHECK("GatedDeltaNet2Fn chunk preparation");
    if (sp.two_tile) LaunchSplit2RecurAny(q, c, sp.sc, sp.nchunks, psi, phi, s0, stream);
    else LaunchSplitRecurAny(q, c, sp.nseg, sp.sc, sp.nchunks, psi, phi, s0, stream);
    XM_LAUNCH_CHECK("GatedDeltaNet2Fn split recurrence");
    const int lds = 2 * 16 * (KT * 16 + 4) * static_cast<int>(sizeof(float));   // two S buffers (combine)
    EnsureDynamicLds(reinterpret_cast<const void *>(&Gdn2SplitCombineKernel), lds);
    EnsureDynamicLds(reinterpret_cast<const void *>(&Gdn2SplitCorrectKernel<1>), lds / 2);
    EnsureDynamicLds(reinterpret_cast<const void *>(&Gdn2SplitCorrectKernel<16>), lds / 2);
    // two segments with no final state: segment 0's final state (in s0) is
    // segment 1's start, and there is nothing to combine
    const bool direct = sp.nseg == 2 && p.final_state == nullptr;
    if (!direct) {
        XM_NOTE_LAUNCH("Gdn2SplitCombineKernel", {}, );
        hipLaunchKernelGGL(Gdn2SplitCombineKernel, dim3(static_cast<unsigned>(rows * VT)), dim3(512), lds, stream, q,
                           sp.nseg, phi, s0, sst);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn split combine");
    }
    // the longest segment s >= 1 (segment 1 of two is the shorter)
    const int seglen = sp.nseg == 2 ? std::min(sp.sc, sp.nchunks - sp.sc) : sp.sc;
    if (KT <= 32 && static_cast<long long>(p.nheads) * p.dv < (1LL << 25) &&
        static_cast<long long>(p.dk) * p.dv < (1LL << 29)) {
        // the state in each wave's registers: blocks of cpw chunks, about two
        // workgroups per CU (1 x 16384 x 8 heads at 256 x 256: 24 chunks per
        // workgroup; 4, 8 and 12 measured the same).  Against the staged
        // kernel below (interleaved A/B): 1 x 16384 x 8 heads at 256 x 256
        // 1.143 -> 1.082 ms, 1 x 8192 x 4 heads at 128 x 128 0.1507 ->
        // 0.1423, 2 x 2048 x 4 heads at 320 x 64 0.1379 -> 0.1358.  The staged
        // kernel remains for states or output rows past the 32-bit offsets.
        const long long vg = (VT + 3) / 4;
        const int cpw = static_cast<int>(
            std::max(1LL, std::min<long long>(std::min(32, seglen), rows * vg * (sp.nchunks - sp.sc) / (2LL * DeviceCus()))));
        const int ncb = (seglen + cpw - 1) / cpw;
        const long long wblocks = static_cast<long long>(sp.nseg - 1) * rows * vg * ncb;
        if (wblocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
        XM_NOTE_LAUNCH("Gdn2SplitCorrectRegKernel", {}, );
        auto kern = KT <= 8 ? Gdn2SplitCorrectRegKernel<8> : KT <= 16 ? Gdn2SplitCorrectRegKernel<16>
                  : KT <= 24 ? Gdn2SplitCorrectRegKernel<24> : Gdn2SplitCorrectRegKernel<32>;
        hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(wblocks)), dim3(256), 0, stream, q, sp.sc, ncb, cpw,
                           sp.nchunks, psi, sst, direct ? s0 : nullptr);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn split correction");
        return;
    }
    // groups of four chunks per segment s >= 1
    const int ncg = (seglen + 3) / 4;
    const long long cblocks = rows * VT * (sp.nseg - 1) * ncg;
    if (cblocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "GatedDeltaNet2Fn launch exceeds the grid limit");
    XM_NOTE_LAUNCH("Gdn2SplitCorrectKernel", {}, );
    // at most four 4-wave workgroups per CU: all resident at once with 112 VGPRs
    const bool overlap = cblocks <= 4LL * DeviceCus();
    hipLaunchKernelGGL(overlap ? Gdn2SplitCorrectKernel<16> : Gdn2SplitCorrectKernel<1>,
                       dim3(static_cast<unsigned>(cblocks)), dim3(256), lds / 2, stream, q, sp.sc, ncg, sp.nchunks, psi,
                       sst, direct ? s0 : nullptr);
    XM_LAUNCH_CHECK("GatedDeltaNet2Fn split correction");
}

// Scratch of one call for a budget of `cap` bytes: the chunks per window and
// sequence (at most 128, fewer when the budget is smaller; 0 when one chunk
// does not fit) and the bytes of the prepared blocks, of the state carried
// between windows (only when a sequence can span several windows) and, for
// packed sequences, of the per-window block offsets.  A window holds chunks
// [c0, c0 + win) of every sequence.  Unpacked, that is win blocks per (b, h).
// Packed (batch sequences along one row of seqlen tokens; no sequence is
// longer than the row), a window's blocks per head are the sequences' chunks
// in it, stored one sequence after the other: at most min(win * batch,
// ceil(seqlen / 16) + batch) of them (each sequence's last chunk may be
// partial); sequence b's start at offs[w][b], [nwin][batch + 1] ints.
struct WindowPlan {
    int win = 0;
    int nchunks = 0;   // sequence-local chunks the windows step over
    int slots = 0;     // blocks per head of one window
    size_t blocks = 0, carry = 0, offsets = 0;
    size_t total() const { return blocks + carry + offsets; }
};

WindowPlan PlanWindows(int batch, int seqlen, int nheads, int dk, int dv, bool packed, size_t cap) {
    const ChunkConfig c = ChooseChunk(dk, static_cast<long long>(batch) * nheads * ((dv + 15) / 16));
    const size_t rows = static_cast<size_t>(packed ? 1 : batch) * nheads;
    const size_t per_block = rows * BlockFloats(c.kpw, c.ks) * sizeof(float);
    const size_t carry = Align256(static_cast<size_t>(batch) * nheads * dk * dv * sizeof(float));
    const int nchunks = (seqlen + kC - 1) / kC;
    const long long all_blocks = static_cast<long long>(nchunks) + batch;   // packed: every sequence's chunks
    auto make = [&](int win, bool with_carry) {
        WindowPlan w;
        w.win = win;
        w.nchunks = nchunks;
        w.slots = packed ? static_cast<int>(std::min<long long>(static_cast<long long>(win) * batch, all_blocks)) : win;
        w.blocks = Align256(per_block * w.slots);
        w.carry = with_carry ? carry : 0;
        const size_t nwin = (nchunks + win - 1) / win;
        w.offsets = packed ? Align256(nwin * (static_cast<size_t>(batch) + 1) * sizeof(int)) : 0;
        return w;
    };
    int win0 = std::min(nchunks, kWindowChunks);
    if (!packed && GetOverride(kOverrideGdn2Windowed) != 1) {
        // Windows of up to 128 MiB of blocks, balanced in length: fewer
        // launches, and preparation launches with enough waves to fill the
        // chip (a 128-chunk window of a few heads is about one wave per SIMD,
        // latency-bound).  Measured against 128-chunk windows (interleaved):
        // 1 x 8192 x 4 heads at 128 x 128 0.503 -> 0.452 ms; 1 x 16384 x 16
        // at 64 x 64 0.953 -> 0.897; 2 x 8192 x 8 at 128 x 128 0.584 ->
        // 0.564; 1 x 16384 x 8 at 256 x 256 1.615 -> 1.545 (four windows of
        // 107 MB; two of 214 MB took 1.745, their blocks falling out of the
        // 256 MB last-level cache before the recurrence reads them).
        const size_t fit = std::min<size_t>((size_t{128} << 20) / per_block, static_cast<size_t>(nchunks));
        if (fit > static_cast<size_t>(win0)) {
            const int nwin = (nchunks + static_cast<int>(fit) - 1) / static_cast<int>(fit);
            win0 = (nchunks + nwin - 1) / nwin;
        }
    }
    WindowPlan w = make(win0, win0 < nchunks);
    if (packed && win0 < nchunks && GetOverride(kOverrideGdn2Windowed) == 0) {
        // The host does not know the sequences' lengths, so it steps through
        // windows up to the row's length, the later ones empty when the
        // sequences are shorter: each costs two launch gaps.  One window over
        // every chunk avoids them; taken when its blocks stay within twice
        // the windowed ones or 512 MiB (with sequences of at most 2048
        // tokens on average the windowed plan already holds every chunk).
        const WindowPlan one = make(nchunks, false);
        if (one.blocks <= std::max<size_t>(2 * w.blocks, size_t{512} << 20) && one.total() <= cap) return one;
    }
    if (w.total() <= cap) return w;
    // shorter windows (the carry is then always needed): the largest that fits
    for (int win = win0 - 1; win >= 1; --win) {
        w = make(win, true);
        if (w.total() <= cap) return w;
    }
    return WindowPlan{};
}

// Packed sequences: for every window w, offs[w][b] = the chunks in [w win,
// (w + 1) win) of sequences 0..b-1 (b = 0..n): where sequence b's blocks of
// window w start.  An empty sequence, which no recurrence workgroup visits,
// passes its initial state (zeros without one) to final_state here.  One
// workgroup.
__global__ __launch_bounds__(256) void Gdn2PackedChunksKernel(GatedDeltaNet2Params p, int *offs, int win, int nwin) {
    __shared__ int part[256];
    const int n = p.batch, tid = threadIdx.x;
    const int per = (n + 255) / 256;
    const int b0 = min(n, tid * per), b1 = min(n, b0 + per);
    auto chunks = [&](int b) {
        size_t tok0;
        int T;
        PackedRange(p, b, tok0, T);
        return (T + kC - 1) / kC;
    };
    for (int w = 0; w < nwin; ++w) {   // workgroup-uniform
        int *const off = offs + static_cast<size_t>(w) * (n + 1);
        auto in_window = [&](int b) { return min(max(chunks(b) - w * win, 0), win); };
        int sum = 0;
        for (int b = b0; b < b1; ++b) sum += in_window(b);
        part[tid] = sum;
        __syncthreads();
        if (tid == 0) {   // exclusive prefix of the 256 partial sums
            int acc = 0;
            for (int i = 0; i < 256; ++i) {
                const int v = part[i];
                part[i] = acc;
                acc += v;
            }
            off[n] = acc;
        }
        __syncthreads();
        int acc = part[tid];
        for (int b = b0; b < b1; ++b) {
            off[b] = acc;
            acc += in_window(b);
        }
        __syncthreads();   // part is rewritten by the next window
    }
    if (p.final_state != nullptr) {
        const size_t hkv = static_cast<size_t>(p.nheads) * p.dk * p.dv;
        for (int b = 0; b < n; ++b) {   // workgroup-uniform
            if (chunks(b) > 0) continue;
            float *dst = p.final_state + static_cast<size_t>(b) * hkv;
            const float *src = p.initial_state != nullptr ? p.initial_state + static_cast<size_t>(b) * hkv : nullptr;
            for (size_t i = tid; i < hkv; i += 256) dst[i] = src != nullptr ? src[i] : 0.0f;
        }
    }
}

}  // namespace

size_t GatedDeltaNet2ChunkScratchBytes(int batch, int seqlen, int nheads, int dk, int dv, bool packed, size_t cap,
                                       bool allow_split) {
    if (dk > kGdn2ChunkKeyLimit) return 0;
    const SplitPlan sp = allow_split ? PlanSplit(batch, seqlen, nheads, dk, dv, packed, cap) : SplitPlan{};
    if (sp.nseg > 0) return sp.total();
    const WindowPlan w = PlanWindows(batch, seqlen, nheads, dk, dv, packed, cap);
    return w.win == 0 ? SIZE_MAX : w.total();
}

bool LaunchGatedDeltaNet2Chunked(const GatedDeltaNet2Params &p, void *scratch, size_t scratch_bytes, void *stream_v) {
    if (GetOverride(kOverrideGdn2Path) == 1) return false;
    if (p.dk > kGdn2ChunkKeyLimit) return false;
    // the recurrence's 32-bit buffer offsets span 16 tokens of [B,T,H,V]
    if (static_cast<long long>(p.nheads) * p.dv >= (1LL << 25)) return false;
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    GatedDeltaNet2Params q = p;
    q.pairwise_only = GetOverride(kOverrideGdn2Pairwise) != 0;
    auto a16 = [](const void *x) { return (reinterpret_cast<uintptr_t>(x) & 15u) == 0; };
    q.vec4_keys = p.dk % 4 == 0 && a16(p.q) && a16(p.k) && a16(p.g) && a16(p.beta);
    const ChunkConfig c = ChooseChunk(p.dk, static_cast<long long>(p.batch) * p.nheads * ((p.dv + 15) / 16));
    const int kq = c.kpw * c.ks;
    const bool packed = p.cu_seqlens != nullptr;
    const SplitPlan sp = PlanSplit(p.batch, p.seqlen, p.nheads, p.dk, p.dv, packed, scratch_bytes);
    if (sp.nseg > 0 && scratch != nullptr) {
        LaunchSplit(q, c, sp, static_cast<char *>(scratch), stream);
        return true;
    }
    const WindowPlan plan = PlanWindows(p.batch, p.seqlen, p.nheads, p.dk, p.dv, packed, scratch_bytes);
    if (plan.win == 0 || plan.total() > scratch_bytes || scratch == nullptr)
        throw Error(XM_ERR_ALLOC, "GatedDeltaNet2Fn: the scratch buffer is smaller than the call needs");
    const int win = plan.win, nchunks = plan.nchunks;
    // rows of a window's prepared blocks: (b, h), or h for packed sequences
    const size_t heads = static_cast<size_t>(packed ? 1 : p.batch) * p.nheads;
    char *base = static_cast<char *>(scratch);
    q.prepared = reinterpret_cast<float *>(base);
    float *const carry = plan.carry > 0 ? reinterpret_cast<float *>(base + plan.blocks) : nullptr;
    int *offs = nullptr;
    if (packed) {
        offs = reinterpret_cast<int *>(base + plan.blocks + plan.carry);
        q.state = carry;
        q.chunk_off = offs;
        XM_NOTE_LAUNCH("Gdn2PackedChunksKernel", {}, );
        hipLaunchKernelGGL(Gdn2PackedChunksKernel, dim3(1), dim3(256), 0, stream, q, offs, win,
                           (nchunks + win - 1) / win);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn packed chunk offsets");
    }
    for (int c0 = 0; c0 < nchunks; c0 += win) {
        // packed: this window's block offsets, and plan.slots blocks per head
        if (packed) q.chunk_off = offs + static_cast<size_t>(c0 / win) * (p.batch + 1);
        const int wn = packed ? plan.slots : std::min(win, nchunks - c0);
        const bool first = c0 == 0, last = c0 + wn >= nchunks;
        XM_NOTE_LAUNCH("Gdn2ChunkPrepKernel", {}, );
        LaunchPrep(c, q, c0, wn, static_cast<long long>(heads) * wn, stream);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn chunk preparation");
        if (packed)   // the kernel picks each sequence's state buffers itself
            LaunchRecurAny(q, c, c0, wn, kq, nullptr, nullptr, stream);
        else
            LaunchRecurAny(q, c, c0, wn, kq, first ? p.initial_state : carry, last ? p.final_state : carry, stream);
        XM_LAUNCH_CHECK("GatedDeltaNet2Fn chunk recurrence");
    }
    return true;
}

}  // namespace xm
