// Plain-old-data launch parameters passed from the host layer to the HIP
// launchers.  Tensors are dense row-major fp32 in the layouts documented on
// each field; index arithmetic in the kernels is 64-bit where a product of
// dimensions can exceed 2^31.
#pragma once

#include <cstddef>
#include <cstdint>

#include "xmetai_recurrent.h"

namespace xm {

// SelectiveScanFn (reference parameter block: selective_scan.h:26-69).
struct SelectiveScanParams {
    // Data tensors (u, delta, variable B/C, out) hold elements of in_type;
    // weights (A, D, delta_bias, constant B/C) and last_state are fp32.
    const void *u;           // [batch, dim, seqlen]
    const void *delta;       // [batch, dim, seqlen]
    const float *A;          // [dim, dstate]
    const void *B;           // b_var ? [batch, groups_b, dstate, seqlen] : [dim, dstate] (fp32)
    const void *C;           // c_var ? [batch, groups_c, dstate, seqlen] : [dim, dstate] (fp32)
    const float *D;          // [dim] or nullptr
    const float *delta_bias; // [dim] or nullptr
    void *out;               // [batch, dim, seqlen]
    int in_type;             // XM_ELEM_FLOAT, XM_ELEM_FLOAT16 or XM_ELEM_BFLOAT16
    float *last_state;       // [batch, dim, dstate]: h after the last token, or nullptr
    int batch, dim, seqlen, dstate;
    int b_var, c_var;
    int groups_b;            // n_groups (from B; 1 when B is constant)
    int groups_c;            // C.shape[1] when C is variable
    int dim_per_group;       // dim / groups_b
    int delta_softplus;
};

// GatedDeltaNet2Fn (reference parameter block: gated_deltanet2.h:13-40).
struct GatedDeltaNet2Params {
    const float *q, *k, *g, *beta;  // [batch, seqlen, nheads, dk]
    const float *v, *w;             // [batch, seqlen, nheads, dv]
    const float *initial_state;     // [batch, nheads, dk, dv] or nullptr
    float *out;                     // [batch, seqlen, nheads, dv]
    float *final_state;             // [batch, nheads, dk, dv]: S after the last token, or nullptr
    float *state;                   // carry between token chunks, [batch, nheads, dk, dv]
    float *prepared;                // [batch*nheads, chunk_cap, 4, dk_pad]: khat, beta*khat*d, qhat*d, d (d = exp(g))
    float *prep_qk;                 // [batch*nheads, chunk_cap]: qhat . khat
    int batch, seqlen, nheads, dk, dv;
    int dk_pad;                     // dk rounded up to the recurrence's key tiling
    int chunk_cap;                  // tokens per preparation chunk (<= 1024)
    int l2norm;
    float scale;
    int pairwise_only;              // chunked path: take the pairwise decay products in every chunk (test switch)
    int vec4_keys;                  // chunked path: dk % 4 == 0 and q, k, g, beta 16-byte aligned
    // Packed sequences: [batch + 1] token offsets along a single row of
    // seqlen tokens (the tensors' batch dimension is 1), or nullptr.
    const int64_t *cu_seqlens;
    // Chunked path with packed sequences: [batch + 1] prefix sums of the
    // sequences' 16-token chunk counts (device scratch), or nullptr.
    const int *chunk_off;
};

// Mamba3SisoFn (reference parameter block: mamba3_siso.h:10-36).
struct Mamba3SisoParams {
    const float *Q, *K;             // [batch, seqlen, nheads_qk, n]
    const float *V;                 // [batch, seqlen, nheads, p]
    const float *ADT, *DT, *Trap;   // [batch, nheads, seqlen]
    const float *Q_bias, *K_bias;   // [nheads, n]
    const float *Angles;            // [batch, seqlen, nheads, a]
    const float *D;                 // [nheads] or nullptr
    const float *Z;                 // [batch, seqlen, nheads, p] or nullptr
    float *out;                     // [batch, seqlen, nheads, p]
    // States (widening): each set all null or all set.  in_*: the state
    // before the first token (S = ssm + v (x) k * the first token's
    // look-ahead); f_*: the state after the last token.
    const float *in_ssm, *in_angle, *in_k, *in_v;   // [batch, nheads, p, n], [.., a], [.., n], [.., p]
    float *f_ssm, *f_angle, *f_k, *f_v;
    // Packed sequences: [batch + 1] token offsets along a single row of
    // seqlen tokens (the tensors' batch dimension is 1), or nullptr.
    const int64_t *cu_seqlens;
    int batch, seqlen, nheads, nheads_qk, n, p, a;
};

// Launchers (defined in the .hip translation units).  They enqueue on
// `stream` and throw xm::Error on a launch failure.
void LaunchSelectiveScan(const SelectiveScanParams &p, void *stream);
// Sequence-parallel form (selective_scan_seg.hip): one workgroup per channel,
// segments of the sequence scanned at once.  Fits: 1 <= dstate <= 256 and one
// batch row of B/C below 2 GiB.
bool SelectiveScanSegFits(const SelectiveScanParams &p);
void LaunchSelectiveScanSeg(const SelectiveScanParams &p, void *stream);
// GatedDeltaNet2Fn host validation (gated_deltanet2_host.cpp): the attribute
// and shape checks of the reference, and the launch parameters of the call.
GatedDeltaNet2Params GatedDeltaNet2Plan(const xm_tensor_t *inputs, size_t n_inputs,
                                        const xm_gated_deltanet2_attrs_t &attrs, float *out, float *final_state);
// Scratch bytes of one call when at most `cap` bytes are available: the
// chunked windows and the token chunks of the dk > 512 path shrink to fit.
// 0 when the call needs none (also when the gdn2_path override runs the
// sequential kernel); SIZE_MAX when not even the smallest layout fits.
// allow_split = false: the windowed plan's bytes, never the sequence split's
// (which keeps every chunk's blocks at once).
size_t GatedDeltaNet2ScratchBytes(int batch, int seqlen, int nheads, int dk, int dv, bool packed,
                                  size_t cap = SIZE_MAX, bool allow_split = true);
// `scratch` holds `scratch_bytes` bytes; the layout is the one
// GatedDeltaNet2ScratchBytes chose for cap = scratch_bytes.
void LaunchGatedDeltaNet2(GatedDeltaNet2Params p, void *scratch, size_t scratch_bytes, void *stream);
// Chunked fp32-MFMA path (dk <= kGdn2ChunkKeyLimit).  Returns false, launching nothing, when
// the shape is not one it takes (or the gdn2_path override asks for the sequential kernel).  `scratch` holds
// scratch_bytes >= GatedDeltaNet2ChunkScratchBytes(..., scratch_bytes) bytes: the
// prepared chunk vectors of one window of up to 2048 tokens (shorter windows
// when the bytes are fewer), and the state carried between windows.
// With `packed`, batch is the number of sequences packed along one row of
// seqlen tokens.
size_t GatedDeltaNet2ChunkScratchBytes(int batch, int seqlen, int nheads, int dk, int dv, bool packed = false,
                                       size_t cap = SIZE_MAX, bool allow_split = true);
constexpr int kGdn2ChunkKeyLimit = 512;   // head_k handled by the chunked path
bool LaunchGatedDeltaNet2Chunked(const GatedDeltaNet2Params &p, void *scratch, size_t scratch_bytes, void *stream);
void LaunchMamba3Siso(const Mamba3SisoParams &p, void *stream);
// Chunked fp32-MFMA path (headdim_qk <= 256).  Returns false, launching
// nothing, when the m3_path override asks for the token-by-token kernel.
bool LaunchMamba3SisoChunked(const Mamba3SisoParams &p, void *stream);
// Enqueues a kernel that writes `count` zeros (no memset node in a captured graph).
void LaunchFillZeros(float *dst, size_t count, void *stream);
// Packed sequences: enqueues a kernel that zeros the token rows of out
// ([seqlen][row_floats]) outside every sequence [cu[b], cu[b + 1]) (clamped as
// the operator kernels clamp them); run before the operator's kernels.
void LaunchPackedGaps(float *out, size_t row_floats, const int64_t *cu, int n, int seqlen, void *stream);

}  // namespace xm
