// Mamba3SisoFn forward, chunked form on fp32 MFMA (gfx950, wave64).
//
// The recurrence (reference mamba3_siso_fwd.cu:79-171), per (b,h) with state
// S [P,N]: S *= e^{ADT_t}; y_t = q^_t . S + (D + qk_t gamma_t) v_t;
// S += v_t (x) k^_t w_t, with q^/k^ the rotated q/k, qk_t the unrotated dot
// product and w_t = gamma_t + look_t (gamma_t = DT_t sigmoid(Trap_t), look_t =
// DT_{t+1} (1 - sigmoid(Trap_{t+1})), 0 for the last token).  The decay is a
// scalar per token, so over a chunk of kC = 16 tokens with cum_t the
// inclusive sum of ADT from the chunk start the recurrence unrolls into
// matrix products:
//   y_t    = e^{cum_t} q^_t . S_prev + sum_{s<t} e^{cum_t - cum_s} w_s (q^_t . k^_s) v_s
//            + (D + qk_t gamma_t) v_t
//   S_next = e^{cum_15} S_prev + sum_s e^{cum_15 - cum_s} w_s v_s (x) k^_s
// (equal to the token-by-token recurrence in exact arithmetic).
//
// A workgroup of 8 waves (12 up to 128 keys) owns one (b,h) and 32 state
// rows (two 16-row tiles) and walks the chunks in order.  Waves 0-3 (product
// waves) form the matrix products and keep S^T in MFMA accumulator layout:
// product wave w holds the key blocks [KBW w, KBW (w+1)) of 16 keys; product
// waves 0 and 1 also finish the previous chunk, with the decay mask and the
// q.k sum that product waves 2 and 3 form for them (and, from 192 keys, the
// whole G^T).  The other waves (preparation waves) prepare the next chunk.
// Each SIMD runs one product wave and one or two preparation waves, so the
// preparation's VALU work and the products' MFMA work overlap.  Per chunk, with
// v_mfma_f32_16x16x4_f32 (A[m][k] in lane m+16k, B[k][n] in lane n+16k,
// D[m][n] in lane n+16(m/4), register m%4):
//   G^T = K^ Q^T   over the wave's keys    (partial, summed across the waves)
//   Y   = Q^ S^T   over the wave's keys    (partial, summed across the waves)
//   S^T = e^{cum_15} S^T + K^T V'           (V'_s = e^{cum_15 - cum_s} w_s v_s)
// and, after the barrier, product waves 0 and 1 each finish one 16-row tile
// of the output: Y e^{cum_t} + (G o L) V + diag v, with L_ts = e^{cum_t - cum_s} w_s
// for s < t, then the SiLU(Z) gate and the store.  An S^T tile register is
// exactly the B operand of the Y product (keys 4(lane/16) + register), so the
// state never moves.
//
// Preparation of chunk j+1 (rotated q^ and k^, V, per-token scalars) runs
// while chunk j's products are formed: the q^ / k^ tiles into one of two LDS
// buffers (chunk parity; chunk j's are read by its products), V^T and the
// per-token fields into one of three (chunk j-1's are read by the finishing
// waves); one barrier per chunk.  Lane (pair lane pq, token group tg) of preparation wave w rotates the pairs
// w PPW + PL x + pq for tokens TPL tg .. TPL tg + TPL - 1.  The angle of a
// pair is a prefix sum over the chunk (fp64: the token groups' sums are
// scanned across lanes) on top of the carried wrapped angle, wrapped once per
// token with the reference's period 2 (float)pi (equal to its wrap after every
// step in exact arithmetic; mamba3_siso.hip does the same).  It is kept in
// turns of that period, where an increment tanh(a) dt (float)pi is the exact
// double tanh(a) dt / 2 and the wrap is one fract.  Tokens past the end
// of the sequence are identity tokens: zero q, k and v, zero ADT and w.
//
// States, packed sequences and the look-ahead hand-over are those of the
// token-by-token kernel (mamba3_siso.hip), which remains the path under the
// m3_path override.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "mamba3_math.h"
#include "xm_hip.h"
#include "xm_matrix.h"
#include "xm_params.h"

namespace xm {
namespace {

using namespace m3;

constexpr int kC = 16;          // tokens per chunk
constexpr int kRows = 32;       // state rows per workgroup (two 16-row tiles)
constexpr int kBufs = 3;        // chunk buffers: preparing j+1, products of j, finishing j-1
// Row stride (floats) of the [key][token] k^T and [row][token] V^T tiles.
// LDS bank conflicts of the kernel's access patterns, measured per access on
// gfx950 (SQ_LDS_BANK_CONFLICT of a probe issuing each pattern), pitch 20
// against 24: V^T 4-byte stores, 32 rows x 2 tokens per wave, 6 and 14 (8
// rows x 8 tokens: 0 at 24); 16-byte reads of 16 rows x 4 tokens 4 and 0;
// k^T 8-byte stores, 8 pair rows x 8 token pairs per wave, 4 and 12, 0 with
// the k^T tile's 4-token groups XOR-swizzled by (row >> 2) & 3 (KtCol).
constexpr int kTS = kC + 8;
// Physical column of token t in row r of the k^T tile: its 4-token group
// XOR (r >> 2) & 3, so a group's 4 tokens stay contiguous for 16-byte reads.
__device__ __forceinline__ int KtCol(int r, int t) { return (((t >> 2) ^ ((r >> 2) & 3)) << 2) | (t & 3); }

template <int KBW, int NW, int NPW>   // 16-key blocks per product wave, product waves, preparation waves
struct M3CLayout {
    static constexpr int NT = 64 * (NW + NPW);   // threads
    static constexpr int NP = 16 * NW * KBW;     // padded headdim_qk
    static constexpr int PPW = NP / (2 * NPW);   // pairs per preparation wave
    static constexpr int PL = PPW % 16 == 0 ? 16 : 8;   // pair lanes per token group
    static constexpr int PB = PPW / PL;          // pairs per lane
    static constexpr int TG = 64 / PL;           // token groups (4 rows, or 8 half rows)
    static constexpr int TPL = kC / TG;          // tokens per lane
    static constexpr int VPT = kRows * kC / (64 * NPW);   // V values per preparation thread
    // Row stride of the [token][key] q^ tile, 8 floats of padding (NP + 8 is 8
    // modulo 16): row-strided 16-byte accesses on gfx950 run without bank
    // conflicts when the row pitch in floats is 8 times an odd number
    // (measured: pitch 132 doubles both the preparation's paired 8-byte
    // writes, 15.8 against 7.9 LDS cycles per instruction, and the products'
    // 16-byte reads, 7.9 against 4.0).
    static constexpr int QS = NP + 8;
    // A chunk's tiles (floats), double-buffered by chunk parity: only the
    // chunk's products and the next chunk's preparation touch them, and in
    // loops unrolled by two the parity, so every tile address, is a
    // compile-time offset from one per-lane base.
    static constexpr int oQ = 0;                      // q^   [kC][QS]
    static constexpr int oKT = oQ + kC * QS;          // k^T  [NP][kTS]
    static constexpr int oK = oKT + NP * kTS;         // k^   [kC][QS] (KCOPY)
    // A chunk's V^T and per-token fields, in three buffers (the finishing
    // waves read them one chunk later).
    static constexpr int oVT = 0;                     // V^T  [kRows][kTS]
    static constexpr int oCum = oVT + kRows * kTS;    // cum_t
    static constexpr int oEcum = oCum + kC;           // e^{cum_t}
    static constexpr int oW = oEcum + kC;             // w_t = gamma_t + look_t
    static constexpr int oGam = oW + kC;              // gamma_t
    static constexpr int oCs = oGam + kC;             // e^{cum_15 - cum_t} w_t (the update's V' scale)
    static constexpr int oQK = oCs + kC;              // partial q.k per preparation wave [NPW][kC]
    // formed once per chunk for both finishing waves, by product waves 2 and 3
    // while the chunk's products run: the decay mask L_ts = e^{cum_t - cum_s}
    // w_s in the finishing MFMA's A layout (lane t + 16 g, register k: s = 4 g
    // + k; s >= t selected away at use) and D + qk_t gamma_t with qk_t the sum
    // of the q.k partials
    static constexpr int oLm = oQK + NPW * kC;        // [64 lanes][4]
    static constexpr int oDg = oLm + 256;             // D + qk_t gamma_t [kC]
    static constexpr int kSmall = oDg + kC;
    // partial products per parity: [NW][3 tiles: G^T, Y rows 0-15, Y rows 16-31][64 lanes][4]
    static constexpr int kPart = NW * 3 * 64 * 4;
    // k^ also in [token][key] order where LDS holds it (up to 256 keys): the
    // G^T product's A operands then come as one 16-byte read per key block
    // (the q^ tile's conflict-free pattern) instead of four 4-byte reads of k^T
    // (2 conflict cycles each)
    static constexpr bool KCOPY = sizeof(float) * (2 * (oK + kC * QS) + kBufs * kSmall + 2 * kPart) <= 160 * 1024;
    static constexpr int kBig = oK + (KCOPY ? kC * QS : 0);
    static constexpr int oBig = 0, oSmall = 2 * kBig, oPart = oSmall + kBufs * kSmall;
    static constexpr size_t kBytes = sizeof(float) * (oPart + 2 * kPart);
    static_assert(kBig % 4 == 0 && kSmall % 4 == 0 && QS % 4 == 0 && kTS % 4 == 0, "16-byte aligned tiles");
    static_assert(kBytes <= 160 * 1024, "LDS budget");
    static_assert(PPW % 8 == 0 && PB * PL == PPW && TPL * TG == kC && VPT * 64 * NPW == kRows * kC, "lane mapping");
    static_assert(VPT * NPW == 8 && kRows == 32 && kC == 16, "V^T: 4 row blocks x 2 token blocks of 8 x 8");
};

// Cross-row moves of one fp64 value per lane with the gfx950 lane-swap
// instructions (rows are 16-lane groups r0..r3):
// permlane16_swap(x, x) -> {[x0, x0, x2, x2], [x1, x1, x3, x3]},
// permlane32_swap(x, x) -> {[x0, x1, x0, x1], [x2, x3, x2, x3]}.
struct D2 {
    double a, b;
};
__device__ __forceinline__ D2 Swap16(double x) {
    const unsigned lo = static_cast<unsigned>(__double_as_longlong(x));
    const unsigned hi = static_cast<unsigned>(static_cast<unsigned long long>(__double_as_longlong(x)) >> 32);
    const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return {__longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(h[0]) << 32) | l[0])),
            __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(h[1]) << 32) | l[1]))};
}
__device__ __forceinline__ D2 Swap32(double x) {
    const unsigned lo = static_cast<unsigned>(__double_as_longlong(x));
    const unsigned hi = static_cast<unsigned>(static_cast<unsigned long long>(__double_as_longlong(x)) >> 32);
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    return {__longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(h[0]) << 32) | l[0])),
            __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(h[1]) << 32) | l[1]))};
}
// Exclusive prefix over the rows: [0, a0, a0 + a1, (a0 + a1) + a2] for row values a_r.
__device__ __forceinline__ double RowExclusiveScan(double a, int row) {
    const D2 p = Swap16(a);                 // [a0, a0, a2, a2], [a1, a1, a3, a3]
    const double pair = p.a + p.b;          // [a0+a1, a0+a1, a2+a3, a2+a3]
    const double e1 = (row & 1) ? p.a : 0.0;
    const double lo = Swap32(pair).a;       // a0 + a1 in every row
    return row >= 2 ? lo + e1 : e1;
}
// Exclusive prefix over 8 token groups laid out as half rows (lane l holds
// group 2 (l / 16) + (l / 8) % 2): the partner half row by DPP row_ror:8,
// then the row sums across rows.
__device__ __forceinline__ double DppRor8(double x) {
    const long long v = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x128, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_mov_dpp(static_cast<int>(v >> 32), 0x128, 0xf, 0xf, true);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}
__device__ __forceinline__ double HalfRowExclusiveScan(double a, int lane);
// Row 3's value in every row.
__device__ __forceinline__ double RowBroadcast3(double x) {
    return Swap16(Swap32(x).b).b;           // [x2, x3, x2, x3] -> [x3, x3, x3, x3]
}
__device__ __forceinline__ double HalfRowExclusiveScan(double a, int lane) {
    const double partner = DppRor8(a);
    const bool upper = (lane & 8) != 0;
    return RowExclusiveScan(a + partner, lane >> 4) + (upper ? partner : 0.0);
}

// Inclusive prefix sum over the 16 lanes of each row (DPP row shifts; a lane
// whose source is outside the row adds 0).
__device__ __forceinline__ float RowInclusiveScan16(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, false));   // row_shr:1
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xf, 0xf, false));   // row_shr:2
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xf, 0xf, false));   // row_shr:4
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xf, 0xf, false));   // row_shr:8
    return x;
}

// LONG: some tensor's token rows of one sequence span 2 GiB or more, beyond a
// buffer descriptor's 32-bit range; every chunk then reads and writes through
// descriptors that start at its own first token.
// HASZ: a Z input (the SiLU gate); without one the finishing waves issue no Z
// loads and no gate.
template <int KBW, int NW, int NPW, bool LONG, bool HASZ>
__global__ __launch_bounds__(64 * (NW + NPW)) void Mamba3ChunkKernel(Mamba3SisoParams p) {
    using L = M3CLayout<KBW, NW, NPW>;
    static_assert(NW == 4, "product waves 0 and 1 finish, 2 and 3 take shared work off them");
    constexpr int NT = L::NT;
    constexpr int PPW = L::PPW, PL = L::PL, PB = L::PB, TPL = L::TPL, VPT = L::VPT, QS = L::QS;

    extern __shared__ __attribute__((aligned(16))) float smem[];
    float *part = smem + L::oPart;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool product_wave = wave < NW;
    const int w = product_wave ? wave : wave - NW;   // index within the role
    const int i16 = lane & 15, g4 = lane >> 4;
    const int N = p.n, P = p.p, A = p.a, H = p.nheads;
    const int half_n = N / 2;
    const int nrb = (P + kRows - 1) / kRows;
    // the nrb workgroups of one (b,h) prepare the same token vectors: keep them on one XCD
    const int wg = XcdLocalBlock(blockIdx.x, gridDim.x);
    const int rb = wg % nrb;
    const int bh = wg / nrb;
    const int b = bh / H, h = bh % H;
    const int gq = h / (H / p.nheads_qk);
    const int r0 = rb * kRows;
    const float dval = p.D ? p.D[h] : 0.0f;
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
    // The offsets come from a vector load: make the sequence's range
    // wave-uniform so the buffer descriptors built from it stay in SGPRs.
    T = __builtin_amdgcn_readfirstlane(T);
    tok0 = Uniform64(tok0);
    sbase = Uniform64(sbase);
    const float *dtr = p.DT + sbase;
    const float *trr = p.Trap + sbase;
    const float *adr = p.ADT + sbase;
    const size_t q_stride = static_cast<size_t>(p.nheads_qk) * N;
    const float *qbase = p.Q + (tok0 * p.nheads_qk + gq) * N;
    const float *kbase = p.K + (tok0 * p.nheads_qk + gq) * N;
    const size_t a_stride = static_cast<size_t>(H) * A;
    const float *abase = p.Angles + (tok0 * H + h) * A;
    const size_t v_stride = static_cast<size_t>(H) * P;
    const size_t vbase = (tok0 * H + h) * P;   // also the output / Z base

    // ---- preparation lanes: pairs w PPW + PL x + pq, tokens TPL tg + s.  Inputs
    // are read with raw buffer loads through per-chunk descriptors that end at
    // the sequence's last token, so tokens past the end, padded pairs (keys
    // >= N) and pairs without an angle (>= A) read zeros with no branch:
    // zero angle increments, zero q/k (padded pairs) and zero DT/ADT/V (a
    // zero w and v make a token past the end an identity token).
    const int pq = lane % PL, tg = lane / PL;
    int pr[PB], qoff[PB][TPL], aoff[PB][TPL];
    float2 qbias[PB], kbias[PB];
    double carry[PB];   // wrapped angle after the last prepared token, in turns of the wrap period
#pragma unroll
    for (int x = 0; x < PB; ++x) {
        pr[x] = w * PPW + PL * x + pq;
        const bool real = pr[x] < half_n, rot = pr[x] < A;
        const int pc = min(pr[x], half_n - 1);
        const float2 qb = *reinterpret_cast<const float2 *>(p.Q_bias + static_cast<size_t>(h) * N + 2 * pc);
        const float2 kb = *reinterpret_cast<const float2 *>(p.K_bias + static_cast<size_t>(h) * N + 2 * pc);
        qbias[x] = real ? qb : make_float2(0.0f, 0.0f);
        kbias[x] = real ? kb : make_float2(0.0f, 0.0f);
        carry[x] = (p.in_angle != nullptr && rot) ? static_cast<double>(p.in_angle[static_cast<size_t>(bh) * A + pr[x]]) * kInvTwoPiF : 0.0;
#pragma unroll
        for (int s = 0; s < TPL; ++s) {
            qoff[x][s] = real ? ((TPL * tg + s) * static_cast<int>(q_stride) + 2 * pr[x]) * 4 : kOutOfRange;
            aoff[x][s] = rot ? ((TPL * tg + s) * static_cast<int>(a_stride) + pr[x]) * 4 : kOutOfRange;
        }
    }
    // V values: block w + NPW u of 8 rows x 8 tokens (row block % 4, token
    // block / 4), lane l: row l / 8, token l % 8 of the block
    int vrow[VPT], vtok[VPT], voff[VPT];
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const int blk = w + NPW * u;
        vrow[u] = 8 * (blk % 4) + (lane >> 3);
        vtok[u] = 8 * (blk / 4) + (lane & 7);
        voff[u] = r0 + vrow[u] < P ? (vtok[u] * static_cast<int>(v_stride) + r0 + vrow[u]) * 4 : kOutOfRange;
    }
    // Without LONG (the host keeps T * stride * 4 < 2^31): one descriptor per
    // tensor for the whole sequence, ending at its last token; the range
    // check covers the per-lane plus the scalar offset, so a token past the
    // end (and kOutOfRange, which stays below 2^32 with any in-range addend)
    // is out of range.  A lane's place within the chunk is the per-lane
    // offset; the chunk's offset is added to it (off), or, for the
    // preparation's loads (SOFF, all but 192 keys), passed as the scalar
    // offset, which saves a vector add per load (4 x 4096 x 32 heads: 128 keys
    // 0.388 -> 0.371 ms, 64 keys 0.250 -> 0.243, 256 keys 0.772 -> 0.768;
    // 192 keys 0.628 -> 0.639, where it stays off; the output stores and Z
    // loads gain nothing measurable from it).  With LONG each chunk's
    // descriptors start at its first token (the sequence's rows can pass
    // 2 GiB).
    auto seq_bytes = [&](size_t stride) { return static_cast<int>(static_cast<size_t>(T) * stride * 4); };
    // (`rows` tokens from c0: DT and Trap reach one token into the next chunk,
    // the look-ahead of the chunk's last token)
    auto chunk_rsrc = [&](const float *base, size_t stride, int c0, int rows = kC) __attribute__((always_inline)) {
        return MakeRsrc(base + static_cast<size_t>(c0) * stride, static_cast<int>(static_cast<size_t>(min(T - c0, rows)) * stride * 4));
    };
    const Rsrc rq = MakeRsrc(qbase, seq_bytes(q_stride));
    const Rsrc rk = MakeRsrc(kbase, seq_bytes(q_stride));
    const Rsrc ra = MakeRsrc(abase, seq_bytes(a_stride));
    const Rsrc rd = MakeRsrc(dtr, T * 4);
    const Rsrc rt = MakeRsrc(trr, T * 4);
    const Rsrc rad = MakeRsrc(adr, T * 4);
    const Rsrc rv = MakeRsrc(p.V + vbase, seq_bytes(v_stride));
    const int qs4 = static_cast<int>(q_stride) * 4, as4 = static_cast<int>(a_stride) * 4, vs4 = static_cast<int>(v_stride) * 4;
    // per-lane offset + chunk offset, added as unsigned (no signed overflow near 2^31)
    auto off = [](int a, int b) { return static_cast<int>(static_cast<unsigned>(a) + static_cast<unsigned>(b)); };
    constexpr bool SOFF = KBW != 3;
    auto ld = [&](Rsrc r, int v, int c) __attribute__((always_inline)) { return SOFF ? BufF(r, v, c) : BufF(r, off(v, c)); };
    auto ld2 = [&](Rsrc r, int v, int c) __attribute__((always_inline)) { return SOFF ? BufF2(r, v, c) : BufF2(r, off(v, c)); };

    // Raw inputs of one chunk, prefetched two chunks ahead into one of two
    // register sets (chunk parity), or, where registers are short (more than
    // 128 keys), one chunk ahead into one set.
    constexpr bool DB = KBW <= 2;
    // The preparation wave that also forms the per-token scalars (gamma, w,
    // the decay scan and its exponentials).  With 8 preparation waves the one
    // on SIMD 2 (waves w of a role sit on SIMD w % 4), the SIMD a per-wave
    // barrier-arrival trace shows with spare issue (4 x 4096 x 32 heads, 128
    // keys: 0.356 -> 0.354 ms against the last wave, on SIMD 3).  With 4 the
    // last: on SIMD 0 instead, where the trace also showed spare issue, it
    // measured slower (64 keys 0.241 -> 0.265 ms, 192 keys 0.623 -> 0.650,
    // 256 keys 0.754 -> 0.764).
    constexpr int kScalarWave = NPW == 8 ? 6 : NPW - 1;
    struct Raw {
        float2 qv[PB][TPL], kv[PB][TPL];
        float ang[PB][TPL], dts[TPL], vreg[VPT];
        float sdt, strap, sadt, sdt1, strap1;   // preparation wave kScalarWave, lane t < kC
    };
    Raw raw0, raw1;
    auto load_prep = [&](int c0, Raw &r) __attribute__((always_inline)) {
        float2 (&qv)[PB][TPL] = r.qv;
        float2 (&kv)[PB][TPL] = r.kv;
        float (&ang)[PB][TPL] = r.ang;
        float (&dts)[TPL] = r.dts;
        float (&vreg)[VPT] = r.vreg;
        const int cq = LONG ? 0 : c0 * qs4, ca = LONG ? 0 : c0 * as4, cv = LONG ? 0 : c0 * vs4, cd = LONG ? 0 : c0 * 4;
        const Rsrc q_ = LONG ? chunk_rsrc(qbase, q_stride, c0) : rq;
        const Rsrc k_ = LONG ? chunk_rsrc(kbase, q_stride, c0) : rk;
        const Rsrc a_ = LONG ? chunk_rsrc(abase, a_stride, c0) : ra;
        const Rsrc d_ = LONG ? chunk_rsrc(dtr, 1, c0, kC + 1) : rd;
        const Rsrc t_ = LONG ? chunk_rsrc(trr, 1, c0, kC + 1) : rt;
        const Rsrc ad_ = LONG ? chunk_rsrc(adr, 1, c0) : rad;
        const Rsrc v_ = LONG ? chunk_rsrc(p.V + vbase, v_stride, c0) : rv;
#pragma unroll
        for (int s = 0; s < TPL; ++s) {
            dts[s] = ld(d_, (TPL * tg + s) * 4, cd);
#pragma unroll
            for (int x = 0; x < PB; ++x) {
                qv[x][s] = ld2(q_, qoff[x][s], cq);
                kv[x][s] = ld2(k_, qoff[x][s], cq);
                ang[x][s] = ld(a_, aoff[x][s], ca);
            }
        }
#pragma unroll
        for (int u = 0; u < VPT; ++u) vreg[u] = ld(v_, voff[u], cv);
        // every preparation wave loads them (same load count on every path); wave kScalarWave uses them
        r.sdt = ld(d_, i16 * 4, cd);
        r.strap = ld(t_, i16 * 4, cd);
        r.sadt = ld(ad_, i16 * 4, cd);
        r.sdt1 = ld(d_, (i16 + 1) * 4, cd);
        r.strap1 = ld(t_, (i16 + 1) * 4, cd);
    };

    // rotated q^ / k^ into the tiles bg, the unrotated q.k, V^T and the
    // per-token scalars of the chunk into bf
    auto prep = [&](float *bg, float *bf, const Raw &r) __attribute__((always_inline)) {
        const float2 (&qv)[PB][TPL] = r.qv;
        const float2 (&kv)[PB][TPL] = r.kv;
        const float (&ang)[PB][TPL] = r.ang;
        const float (&dts)[TPL] = r.dts;
        const float (&vreg)[VPT] = r.vreg;
        float qk[TPL];
#pragma unroll
        for (int s = 0; s < TPL; ++s) qk[s] = 0.0f;
#pragma unroll
        for (int x = 0; x < PB; ++x) {
            double pre[TPL], acc = 0.0;
            // The angle in turns of the wrap period 2 (float)pi (reference
            // :26-28): the increment tanh(a) dt (float)pi is tanh(a) dt / 2
            // turns, exact in double (a product of two floats).
#pragma unroll
            for (int s = 0; s < TPL; ++s) {
                acc += static_cast<double>(0.5f * TanhF(ang[x][s])) * static_cast<double>(dts[s]);
                pre[s] = acc;
            }
            // exclusive prefix of the token groups' sums (lanes pq + PL tg)
            double excl;
            if constexpr (PL == 16) excl = RowExclusiveScan(acc, tg);   // token groups are rows
            else excl = HalfRowExclusiveScan(acc, lane);                 // token groups are half rows
            const double base = carry[x] + excl;
            double th = 0.0;
            float kc0[TPL], kc1[TPL];
#pragma unroll
            for (int s = 0; s < TPL; ++s) {
                th = base + pre[s];
                th = __builtin_amdgcn_fract(th);   // wrap_two_pi (reference :26-28), in turns: th - floor(th), kept below 1
                // a pair without an angle keeps theta = 0: sin 0 = 0, cos 0 = 1
                const float rev = static_cast<float>(th * kRevPerTurn);
                const float sn = __builtin_amdgcn_sinf(rev), c = __builtin_amdgcn_cosf(rev);
                const float2 q = make_float2(qv[x][s].x + qbias[x].x, qv[x][s].y + qbias[x].y);
                const float2 k = make_float2(kv[x][s].x + kbias[x].x, kv[x][s].y + kbias[x].y);
                qk[s] = fmaf(q.x, k.x, fmaf(q.y, k.y, qk[s]));   // unrotated q.k (reference :89-106)
                *reinterpret_cast<float2 *>(bg + L::oQ + (TPL * tg + s) * QS + 2 * pr[x]) =
                    make_float2(q.x * c - q.y * sn, q.x * sn + q.y * c);
                kc0[s] = k.x * c - k.y * sn;
                kc1[s] = k.x * sn + k.y * c;
                if constexpr (L::KCOPY)
                    *reinterpret_cast<float2 *>(bg + L::oK + (TPL * tg + s) * QS + 2 * pr[x]) = make_float2(kc0[s], kc1[s]);
            }
            const int r0k = 2 * pr[x], r1k = 2 * pr[x] + 1;   // this lane's tokens stay in one swizzled group
            if constexpr (TPL == 4) {
                StF4(bg + L::oKT + r0k * kTS + KtCol(r0k, 4 * tg), v4f{kc0[0], kc0[1], kc0[2], kc0[3]});
                StF4(bg + L::oKT + r1k * kTS + KtCol(r1k, 4 * tg), v4f{kc1[0], kc1[1], kc1[2], kc1[3]});
            } else {
                *reinterpret_cast<float2 *>(bg + L::oKT + r0k * kTS + KtCol(r0k, TPL * tg)) = make_float2(kc0[0], kc0[1]);
                *reinterpret_cast<float2 *>(bg + L::oKT + r1k * kTS + KtCol(r1k, TPL * tg)) = make_float2(kc1[0], kc1[1]);
            }
            // the chunk's last token
            if constexpr (PL == 16) {
                carry[x] = RowBroadcast3(th);
            } else {
                // row 3 holds groups 6 (lower half) and 7; the DPP move runs in
                // every lane before the select (a move inside a branch would
                // read inactive lanes)
                const double v = RowBroadcast3(th);
                const double vr = DppRor8(v);
                carry[x] = (lane & 8) ? v : vr;
            }
        }
        // q.k partial over this wave's pairs, per token
#pragma unroll
        for (int s = 0; s < TPL; ++s) {
            float v = qk[s];
            v += DppF<0xB1>(v);    // quad_perm [1,0,3,2]
            v += DppF<0x4E>(v);    // quad_perm [2,3,0,1]
            v += DppF<0x141>(v);   // row_half_mirror: the 8 lanes of a half row
            if constexpr (PL == 16) v += DppF<0x128>(v);   // row_ror:8
            bf[L::oQK + w * kC + TPL * tg + s] = v;   // every lane of the token group holds the sum
        }
#pragma unroll
        for (int u = 0; u < VPT; ++u) bf[L::oVT + vrow[u] * kTS + vtok[u]] = vreg[u];
        if (w == kScalarWave) {
            const float gam = r.sdt * FastSigmoid(r.strap);
            const float look = r.sdt1 * (1.0f - FastSigmoid(r.strap1));   // zero DT past the end
            const float cum = RowInclusiveScan16(r.sadt);   // over the chunk's 16 tokens (lanes 0-15)
            const float cum15 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cum), kC - 1));
            if (lane < kC) {
                bf[L::oCum + lane] = cum;
                bf[L::oEcum + lane] = __expf(cum);
                bf[L::oW + lane] = gam + look;
                bf[L::oGam + lane] = gam;
                bf[L::oCs + lane] = __expf(cum15 - cum) * (gam + look);
            }
        }
    };

    // ---- state: S^T tile (key block kb, row tile pt), lane i16 + 16 g4,
    // register r = S[row r0 + 16 pt + i16][key 16 (KBW w + kb) + 4 g4 + r]
    v4f S[KBW][2];
    {
        const float look0 = (p.in_ssm != nullptr && T > 0) ? dtr[0] * (1.0f - FastSigmoid(trr[0])) : 0.0f;
#pragma unroll
        for (int kb = 0; kb < KBW; ++kb)
#pragma unroll
            for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = r0 + 16 * pt + i16, key = 16 * (KBW * w + kb) + 4 * g4 + r;
                    float v = 0.0f;
                    if (product_wave && p.in_ssm != nullptr && row < P && key < N) {
                        const float vl = p.in_v[static_cast<size_t>(bh) * P + row];
                        const float kl = p.in_k[static_cast<size_t>(bh) * N + key];
                        v = fmaf(vl, kl * look0, p.in_ssm[(static_cast<size_t>(bh) * P + row) * N + key]);
                    }
                    S[kb][pt][r] = v;
                }
    }

    // ---- products of one chunk: partial G^T and Y to LDS, then the state update
    // G^T = K Q^T is summed over all keys: the finishing waves 0 and 1 form it
    // over the first GK0 of their key blocks only, waves 2 and 3 over theirs
    // and the remaining GX of wave w - 2's.  Measured (4 x 4096 x 32 heads,
    // 2 x at 192 and 256 keys): up to 128 keys nothing moves (one block
    // moved: 0.398 -> 0.421 ms, both: 0.431); at 192 and 256 keys all of
    // them move (0.684 -> 0.628, 0.809 -> 0.763 ms; with the A operands as
    // 4-byte k^T reads, before the k^ copy fitted there: 0.711 -> 0.656,
    // 0.822 -> 0.795, one of three or two of four 0.659, 0.806).
    constexpr int GK0 = KBW <= 2 ? KBW : 0, GX = KBW - GK0;
    auto load_qk = [&](const float *bg, int nb0, float (&q)[4], float (&k)[4]) __attribute__((always_inline)) {
        const v4f q4 = LdsF4(bg + L::oQ + i16 * QS + nb0 + 4 * g4);
        v4f k4;
        if constexpr (L::KCOPY) k4 = LdsF4(bg + L::oK + i16 * QS + nb0 + 4 * g4);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int kr = nb0 + 4 * g4 + ks;
            q[ks] = q4[ks];                                       // q^[t = i16][key nb0 + 4 g4 + ks]
            if constexpr (L::KCOPY) k[ks] = k4[ks];               // k^[s = i16][same key]
            else k[ks] = bg[L::oKT + kr * kTS + KtCol(kr, i16)];
        }
    };
    auto products = [&](const float *bg, const float *bf, float *pp) __attribute__((always_inline)) {
        float qa[KBW][4], ka[KBW][4], kt[KBW][4], qx[GX > 0 ? GX : 1][4], kx[GX > 0 ? GX : 1][4];
#pragma unroll
        for (int kb = 0; kb < KBW; ++kb) {
            const int nb0 = 16 * (KBW * w + kb);
            load_qk(bg, nb0, qa[kb], ka[kb]);
            const v4f t4 = LdsF4(bg + L::oKT + (nb0 + i16) * kTS + KtCol(nb0 + i16, 4 * g4));
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) kt[kb][ks] = t4[ks];   // k^[s = 4 g4 + ks][key nb0 + i16]
        }
        if (w >= 2) {
#pragma unroll
            for (int x = 0; x < GX; ++x) load_qk(bg, 16 * (KBW * (w - 2) + GK0 + x), qx[x], kx[x]);
        }
        const v4f cs = LdsF4(bf + L::oCs + 4 * g4);
        const float ecum15 = bf[L::oEcum + kC - 1];
        v4f vt[2];
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) vt[pt] = LdsF4(bf + L::oVT + (16 * pt + i16) * kTS + 4 * g4);

        v4f gp = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < GK0; ++kb)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) gp = Mfma(ka[kb][ks], qa[kb][ks], gp);   // G^T[s][t]
        if (w >= 2) {
#pragma unroll
            for (int kb = GK0; kb < KBW; ++kb)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) gp = Mfma(ka[kb][ks], qa[kb][ks], gp);
#pragma unroll
            for (int x = 0; x < GX; ++x)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) gp = Mfma(kx[x][ks], qx[x][ks], gp);
        }
        v4f yp[2];
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) {
            yp[pt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < KBW; ++kb)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) yp[pt] = Mfma(qa[kb][ks], S[kb][pt][ks], yp[pt]);   // Y[t][row]
        }
        if (GK0 > 0 || w >= 2) StF4(pp + ((w * 3 + 0) * 64 + lane) * 4, gp);
        StF4(pp + ((w * 3 + 1) * 64 + lane) * 4, yp[0]);
        StF4(pp + ((w * 3 + 2) * 64 + lane) * 4, yp[1]);

        // S^T = e^{cum_15} S^T + K^T V',  V'[s][row] = e^{cum_15 - cum_s} w_s v_s[row]
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) {
            float vs[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) vs[r] = vt[pt][r] * cs[r];
#pragma unroll
            for (int kb = 0; kb < KBW; ++kb) {
                S[kb][pt] *= ecum15;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) S[kb][pt] = Mfma(kt[kb][ks], vs[ks], S[kb][pt]);
            }
        }
    };

    // ---- output rows 16 pt .. 16 pt + 15 of the chunk at c0 (product waves 0 and 1)
    const int orow = r0 + 16 * w + i16;
    int ooff[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        ooff[r] = (w < 2 && orow < P) ? ((4 * g4 + r) * static_cast<int>(v_stride) + orow) * 4 : kOutOfRange;
    // Z of the rows a finishing wave stores, loaded before the products so the
    // MFMA work covers the latency.
    const Rsrc rz = MakeRsrc(p.Z != nullptr ? p.Z + vbase : p.out, p.Z != nullptr ? seq_bytes(v_stride) : 0);
    const Rsrc ro = MakeRsrc(p.out + vbase, seq_bytes(v_stride));
    const Rsrc rnone = MakeRsrc(p.out, 0);   // every access dropped
    auto load_z = [&](int c0, float (&zr)[4]) __attribute__((always_inline)) {
        if constexpr (!HASZ) return;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (LONG) zr[r] = BufF(p.Z != nullptr ? chunk_rsrc(p.Z + vbase, v_stride, c0) : rnone, ooff[r]);
            else zr[r] = BufF(rz, off(ooff[r], c0 * vs4));
        }
    };
    // y of chunk c0 (tokens past the end and rows >= P are dropped).  The
    // values stay in their four registers until every store is issued: a
    // store's data register rewritten behind it waits for the store to
    // complete (stores count in vmcnt on gfx950).
    auto store_y = [&](int c0, const float (&y)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (LONG) BufStF(chunk_rsrc(p.out + vbase, v_stride, c0), ooff[r], y[r]);
            else BufStF(ro, off(ooff[r], c0 * vs4), y[r]);
        }
        asm volatile("" ::"v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]));
    };
    auto finish = [&](const float *bf, const float *pp, const float (&zr)[4], float (&y)[4])
                      __attribute__((always_inline)) {
        const int pt = w;
        constexpr int GW0 = GK0 > 0 ? 0 : 2;   // first wave with a G^T partial
        v4f g = LdsF4(pp + ((GW0 * 3) * 64 + lane) * 4), ys = LdsF4(pp + ((1 + pt) * 64 + lane) * 4);
        const v4f dg4 = LdsF4(bf + L::oDg + 4 * g4);   // D + qk_t gamma_t
        const v4f l4 = LdsF4(bf + L::oLm + lane * 4);
#pragma unroll
        for (int w2 = GW0 + 1; w2 < NW; ++w2) g += LdsF4(pp + ((w2 * 3 + 0) * 64 + lane) * 4);   // product waves' partials
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) ys += LdsF4(pp + ((w2 * 3 + 1 + pt) * 64 + lane) * 4);
        const v4f ecum4 = LdsF4(bf + L::oEcum + 4 * g4);
        const v4f vt = LdsF4(bf + L::oVT + (16 * pt + i16) * kTS + 4 * g4);
        // M[t = i16][s = 4 g4 + ks] = G[t][s] e^{cum_t - cum_s} w_s for s < t (A operand)
        float m[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int s = 4 * g4 + ks;
            m[ks] = s < i16 ? g[ks] * l4[ks] : 0.0f;
        }
        // acc[r] (t = 4 g4 + r, this lane's row): e^{cum_t} Y + (D + qk_t gamma_t) v_t
        v4f acc;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(ecum4[r], ys[r], dg4[r] * vt[r]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = Mfma(m[ks], vt[ks], acc);   // + sum_{s<t} M[t][s] v_s
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            y[r] = acc[r];
            if constexpr (HASZ) y[r] *= zr[r] * FastSigmoid(zr[r]);   // silu gate (reference :155-158)
        }
    };

    // What both finishing waves of chunk bf would otherwise each form (the
    // finishing waves' SIMDs carry the most issue): wave 2 sums the q.k
    // partials (in preparation-wave order) into D + qk_t gamma_t, wave 3 forms
    // the decay mask, while the chunk's products run; the chunk is finished
    // after the next barrier.
    auto shared_finish = [&](float *bf) __attribute__((always_inline)) {
        if (w == 2) {
            if (lane < kC) {
                float v = bf[L::oQK + lane];
#pragma unroll
                for (int w2 = 1; w2 < NPW; ++w2) v += bf[L::oQK + w2 * kC + lane];
                bf[L::oDg + lane] = fmaf(v, bf[L::oGam + lane], dval);
            }
        } else if (w == 3) {
            const v4f cum4 = LdsF4(bf + L::oCum + 4 * g4), w4 = LdsF4(bf + L::oW + 4 * g4);
            const float cumt = bf[L::oCum + i16];
            v4f l4;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) l4[ks] = __expf(cumt - cum4[ks]) * w4[ks];
            StF4(bf + L::oLm + lane * 4, l4);
        }
    };

    const int nch = (T + kC - 1) / kC;
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    auto big = [&](auto P) { return smem + L::oBig + decltype(P)::value * L::kBig; };      // chunk parity P
    auto par = [&](auto P) { return part + decltype(P)::value * L::kPart; };
    auto small = [&](int j) { return smem + L::oSmall + (j % kBufs) * L::kSmall; };
    // Each role runs its own loop (the same barriers, in the same order), so
    // the registers one role carries across chunks (the state S; the
    // prefetched inputs and angle carries) never have to coexist, and no wave
    // carries another role's predicated-off work (waves 2 and 3 issue no Z
    // loads or output stores: 0.395 -> 0.387 ms at 4 x 4096 x 32 heads, 128
    // keys).  Iteration j: products of chunk j, finishing of chunk j-1 (waves
    // 0 and 1) or the shared finishing work of chunk j (waves 2 and 3) |
    // prefetch of chunk j+2, preparation of chunk j+1.  Chunk 0's products and
    // the last chunk's finishing are peeled.
    if (nch > 0 && product_wave && w < 2) {   // workgroup-uniform: an empty sequence passes its states through
        __syncthreads();
        // Z of chunk j is loaded in iteration j (before its products) into
        // the register set of j's parity and gated in iteration j + 1, where
        // chunk j is finished.  Loaded in the finishing iteration itself, it
        // came after the previous chunk's output stores, and the wait for it
        // (stores count in vmcnt on gfx950) waited for those stores to
        // complete.  The sets are written only by the Z loads: a zeroing in
        // every iteration landed on registers the previous stores read.
        float za[4] = {0.0f, 0.0f, 0.0f, 0.0f}, zb[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        load_z(0, za);
        products(big(P0{}), small(0), par(P0{}));
        __syncthreads();
        // zl: the set for chunk j's Z; zu: chunk j - 1's, finished here.  The
        // values stay in their four registers until every store is issued: a
        // store's data register rewritten behind it waits for the store to
        // complete (stores count in vmcnt on gfx950).
        // P: chunk j's parity.
        auto iter = [&](int j, auto P, float (&zl)[4], const float (&zu)[4]) __attribute__((always_inline)) {
            using Q = std::integral_constant<int, 1 - decltype(P)::value>;
            load_z(j * kC, zl);
            products(big(P), small(j), par(P));
            float y[4];
            finish(small(j - 1), par(Q{}), zu, y);
            store_y((j - 1) * kC, y);
            __syncthreads();
        };
        for (int j = 1; j < nch; j += 2) {   // unrolled by two for the sets and the parity
            iter(j, P1{}, zb, za);
            if (j + 1 >= nch) break;
            iter(j + 1, P0{}, za, zb);
        }
        float y[4];
        if ((nch - 1) & 1) finish(small(nch - 1), par(P1{}), zb, y);
        else finish(small(nch - 1), par(P0{}), za, y);
        store_y((nch - 1) * kC, y);
    } else if (nch > 0 && product_wave) {   // waves 2 and 3: products and the shared finishing work
        __syncthreads();
        auto step = [&](int j, auto P) __attribute__((always_inline)) {
            products(big(P), small(j), par(P));
            shared_finish(small(j));
            __syncthreads();
        };
        for (int j = 0; j < nch; j += 2) {   // unrolled by two for the parity
            step(j, P0{});
            if (j + 1 >= nch) break;
            step(j + 1, P1{});
        }
    } else if (nch > 0) {
        load_prep(0, raw0);
        if constexpr (DB) load_prep(min(1, nch - 1) * kC, raw1);
        prep(big(P0{}), small(0), raw0);
        if constexpr (!DB) load_prep(min(1, nch - 1) * kC, raw0);
        __syncthreads();
        // unrolled by two for the register sets and the parity (P: chunk j + 1's)
        auto iter = [&](int j, auto P, Raw &ld, const Raw &pr_) __attribute__((always_inline)) {
            if constexpr (DB) load_prep(min(j + 2, nch - 1) * kC, ld);
            prep(big(P), small(j + 1), pr_);
            if constexpr (!DB) load_prep(min(j + 2, nch - 1) * kC, ld);
            __syncthreads();
        };
        if (nch > 1) {
            for (int j = 0;; j += 2) {
                iter(j, P1{}, raw0, DB ? raw1 : raw0);
                if (j + 2 >= nch) break;
                iter(j + 1, P0{}, DB ? raw1 : raw0, raw0);
                if (j + 3 >= nch) break;
            }
        }
        __syncthreads();   // the products of the last chunk
    }

    if (p.f_ssm != nullptr) {
        if (product_wave) {
#pragma unroll
            for (int kb = 0; kb < KBW; ++kb)
#pragma unroll
                for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = r0 + 16 * pt + i16, key = 16 * (KBW * w + kb) + 4 * g4 + r;
                        if (row < P && key < N) p.f_ssm[(static_cast<size_t>(bh) * P + row) * N + key] = S[kb][pt][r];
                    }
        } else if (rb == 0) {
#pragma unroll
            for (int x = 0; x < PB; ++x)
                if (tg == 0 && pr[x] < A)
                    p.f_angle[static_cast<size_t>(bh) * A + pr[x]] = static_cast<float>(carry[x] * kTwoPiF);
        }
        if (tid < kRows && r0 + tid < P) {
            const size_t o = static_cast<size_t>(bh) * P + r0 + tid;
            p.f_v[o] = T > 0 ? p.V[vbase + static_cast<size_t>(T - 1) * v_stride + r0 + tid]
                             : (p.in_v != nullptr ? p.in_v[o] : 0.0f);
        }
        if (rb == 0) {
            // the last chunk's tiles are intact: its k^T column of the last token
            const int tl = T > 0 ? (T - 1) - (nch - 1) * kC : 0;
            const float *kt = smem + L::oBig + ((nch > 0 ? nch - 1 : 0) & 1) * L::kBig + L::oKT;
            for (int i = tid; i < N; i += NT) {
                const size_t o = static_cast<size_t>(bh) * N + i;
                p.f_k[o] = T > 0 ? kt[i * kTS + KtCol(i, tl)] : (p.in_k != nullptr ? p.in_k[o] : 0.0f);
            }
        }
    }
}

template <int KBW, int NW, int NPW, bool LONG, bool HASZ>
void LaunchChunkZ(const Mamba3SisoParams &p, hipStream_t stream) {
    using L = M3CLayout<KBW, NW, NPW>;
    const long long blocks = static_cast<long long>(p.batch) * p.nheads * ((p.p + kRows - 1) / kRows);
    if (blocks > 2147483647LL) throw Error(XM_ERR_INVALID_ARGUMENT, "Mamba3SisoFn launch exceeds the grid limit");
    EnsureDynamicLds(reinterpret_cast<const void *>(&Mamba3ChunkKernel<KBW, NW, NPW, LONG, HASZ>), static_cast<int>(L::kBytes));
    XM_NOTE_LAUNCH("Mamba3ChunkKernel", {}, KBW, NW, NPW, LONG);
    hipLaunchKernelGGL((Mamba3ChunkKernel<KBW, NW, NPW, LONG, HASZ>), dim3(static_cast<unsigned>(blocks)), dim3(L::NT),
                       L::kBytes, stream, p);
}

template <int KBW, int NW, int NPW, bool LONG>
void LaunchChunkL(const Mamba3SisoParams &p, hipStream_t stream) {
    if (p.Z != nullptr) LaunchChunkZ<KBW, NW, NPW, LONG, true>(p, stream);
    else LaunchChunkZ<KBW, NW, NPW, LONG, false>(p, stream);
}

template <int KBW, int NW, int NPW>
void LaunchChunk(const Mamba3SisoParams &p, bool long_rows, hipStream_t stream) {
    if (long_rows) LaunchChunkL<KBW, NW, NPW, true>(p, stream);
    else LaunchChunkL<KBW, NW, NPW, false>(p, stream);
}

}  // namespace

bool LaunchMamba3SisoChunked(const Mamba3SisoParams &p, void *stream_v) {
    if (GetOverride(kOverrideM3Path) == 1) return false;
    // Buffer descriptors hold 32-bit byte sizes.  The token rows of Q/K,
    // Angles and V/Z/out of one sequence below 2 GiB each: one descriptor per
    // tensor for the whole sequence.  From 2 GiB on: per-chunk descriptors
    // (16 token rows each must stay below 2 GiB).
    const size_t widest = std::max({static_cast<size_t>(p.nheads_qk) * p.n, static_cast<size_t>(p.nheads) * p.a,
                                    static_cast<size_t>(p.nheads) * p.p});
    const size_t row_bytes = widest * sizeof(float);
    if (row_bytes * kC >= (size_t{1} << 31)) return false;
    const bool long_rows = static_cast<size_t>(p.seqlen) * row_bytes >= (size_t{1} << 31);
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    // headdim_qk padded to 64, 128, 192 or 256 keys
    if (p.n <= 64) LaunchChunk<1, 4, 4>(p, long_rows, stream);
    else if (p.n <= 128) LaunchChunk<2, 4, 8>(p, long_rows, stream);   // 8 product waves: slower (more partials)
    else if (p.n <= 192) LaunchChunk<3, 4, 4>(p, long_rows, stream);
    else if (p.n <= 256) LaunchChunk<4, 4, 4>(p, long_rows, stream);
    else return false;
    XM_LAUNCH_CHECK("Mamba3SisoFn (chunked)");
    return true;
}

}  // namespace xm
