// GatedDeltaNet2Fn host layer: attribute checks, shape validation, scratch
// and launch.  Mirrors gated_deltanet2_fn_ort.cpp:46-219 of the reference
// (constructor checks in the same order, ValidateInputs and its messages,
// ToIntDim, output shape = v.shape).
//
// Scratch (requested from the caller's allocator, reference :86-111): for
// headdim_k <= 512 the chunked path's prepared blocks of one window of up to
// 128 16-token chunks plus the state carried between windows (packed
// sequences and the sequential kernel take none); above 512 keys the prepared
// per-token vectors of one <=1024-token chunk, the state carried between
// chunks, and above 2048 keys the recurrence's state tiles.  Any headdim_k is
// accepted, as in the reference's generic kernel (gated_deltanet2_fwd.cu:142-233).
//
// Widening: output_final_state = 1, which the reference rejects (:49-51), is
// accepted through xm_gated_deltanet2_forward_states, which also writes the
// state after the last token, [batch, nheads, headdim_k, headdim_v] (the
// layout initial_state takes, so a call can continue where another stopped).
// Widening: has_cu_seqlens = 1 (rejected at :55-57) packs N sequences along
// seqlen: input 7 is cu_seqlens (int64 [N+1]), the tensors have batch 1 and
// the states are [N, nheads, headdim_k, headdim_v]; the fused kernel reads
// each sequence's token range on the device (headdim_k up to 512).
#include <cmath>

#include "xm_common.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr size_t kNumInputs = 7;
constexpr size_t kNumInputsPacked = 8;   // + cu_seqlens

void CheckAttrs(const xm_gated_deltanet2_attrs_t &a) {
    if (a.use_gate_in_kernel != 0)
        Unsupported("GatedDeltaNet2Fn v1 expects pre-applied gate tensors and does not support use_gate_in_kernel");
    if (a.state_v_first != 0) Unsupported("GatedDeltaNet2Fn v1 expects state layout (batch, head, key, value)");
    if (!(a.scale > 0.0f) || !std::isfinite(a.scale)) Invalid("GatedDeltaNet2Fn requires a positive finite scale");
}

struct Plan {
    GatedDeltaNet2Params params{};
    std::vector<int64_t> out_shape;
    size_t scratch = 0;
};

Plan Validate(const std::vector<View> &in, const IndexView *cu, const xm_gated_deltanet2_attrs_t &attrs) {
    const View &q = in[0], &k = in[1], &v = in[2], &g = in[3], &beta = in[4], &w = in[5], &s0 = in[6];
    // ValidateInputs (reference :187-219)
    RequireRank(q, 4, "q");
    RequireRank(k, 4, "k");
    RequireRank(v, 4, "v");
    RequireRank(g, 4, "g");
    RequireRank(beta, 4, "beta");
    RequireRank(w, 4, "w");
    RequireSameShape(q, k, "q", "k");
    RequireSameShape(q, g, "q", "g");
    RequireSameShape(q, beta, "q", "beta");
    if (v.shape[0] != q.shape[0] || v.shape[1] != q.shape[1] || v.shape[2] != q.shape[2])
        Invalid("v batch/seqlen/head dimensions must match q");
    RequireSameShape(v, w, "v", "w");
    // packed sequences: one row of tokens, one state per sequence
    if (cu != nullptr && q.shape[0] != 1)
        Invalid("GatedDeltaNet2Fn with cu_seqlens requires batch 1 (sequences packed along seqlen)");
    const int64_t nstate = cu != nullptr ? cu->count - 1 : q.shape[0];
    if (s0.present()) {
        RequireRank(s0, 4, "initial_state");
        if (s0.shape[0] != nstate || s0.shape[1] != q.shape[2] || s0.shape[2] != q.shape[3] ||
            s0.shape[3] != v.shape[3])
            Invalid(cu != nullptr ? "initial_state must have shape (sequences, head, headdim_k, headdim_v)"
                                  : "initial_state must have shape (batch, head, headdim_k, headdim_v)");
    }
    Plan plan;
    plan.out_shape = v.shape;
    GatedDeltaNet2Params &p = plan.params;
    p.batch = ToIntDim(nstate, cu != nullptr ? "sequences" : "batch");
    p.seqlen = ToIntDim(q.shape[1], "seqlen");
    p.nheads = ToIntDim(q.shape[2], "nheads");
    p.dk = ToIntDim(q.shape[3], "headdim_k");
    p.dv = ToIntDim(v.shape[3], "headdim_v");
    if (cu != nullptr && p.dk > 512) Unsupported("GatedDeltaNet2Fn with cu_seqlens supports headdim_k up to 512");
    p.cu_seqlens = cu != nullptr ? cu->data : nullptr;
    p.q = q.data;
    p.k = k.data;
    p.v = v.data;
    p.g = g.data;
    p.beta = beta.data;
    p.w = w.data;
    p.initial_state = s0.present() ? s0.data : nullptr;
    p.l2norm = attrs.use_qk_l2norm_in_kernel != 0;
    p.scale = attrs.scale;
    plan.scratch = GatedDeltaNet2ScratchBytes(p.batch, p.seqlen, p.nheads, p.dk, p.dv, cu != nullptr);
    return plan;
}

// The views (7 float inputs, plus cu_seqlens when packed) and the plan.
Plan Prepare(const xm_tensor_t *inputs, size_t n_inputs, const xm_gated_deltanet2_attrs_t &attrs) {
    const bool packed = attrs.has_cu_seqlens != 0;
    auto views = MakeViews(inputs, n_inputs, packed ? kNumInputsPacked : kNumInputs, "GatedDeltaNet2Fn", kNumInputs);
    if (!packed) return Validate(views, nullptr, attrs);
    const IndexView cu = MakeIndexView(inputs[kNumInputs], "cu_seqlens");
    return Validate(views, &cu, attrs);
}

void Forward(const xm_tensor_t *inputs, size_t n_inputs, const xm_gated_deltanet2_attrs_t &attrs, float *out,
             float *final_state, void *stream, const xm_allocator_t *alloc) {
    const GatedDeltaNet2Params p = GatedDeltaNet2Plan(inputs, n_inputs, attrs, out, final_state);
    const bool packed = p.cu_seqlens != nullptr;
    size_t bytes = GatedDeltaNet2ScratchBytes(p.batch, p.seqlen, p.nheads, p.dk, p.dv, packed);
    Scratch scratch(alloc, stream);
    void *buf = scratch.TryGet(bytes);
    if (buf == nullptr && bytes > 0) {
        // The sequence split keeps every chunk's blocks at once; when the
        // allocator refuses that, the windowed plan (a window's blocks plus
        // the carried state) runs the same call in less.
        const size_t windowed =
            GatedDeltaNet2ScratchBytes(p.batch, p.seqlen, p.nheads, p.dk, p.dv, packed, SIZE_MAX, false);
        if (windowed >= bytes)
            throw Error(XM_ERR_ALLOC, "scratch allocation of " + std::to_string(bytes) + " bytes failed");
        bytes = windowed;
        buf = scratch.Get(bytes);
    }
    LaunchGatedDeltaNet2(p, buf, bytes, stream);
}

}  // namespace

GatedDeltaNet2Params GatedDeltaNet2Plan(const xm_tensor_t *inputs, size_t n_inputs,
                                        const xm_gated_deltanet2_attrs_t &attrs, float *out, float *final_state) {
    ResetLaunches();
    CheckAttrs(attrs);
    Plan plan = Prepare(inputs, n_inputs, attrs);
    if (out == nullptr) Invalid("output pointer is null");
    const bool want_state = attrs.output_final_state != 0;
    if (want_state && final_state == nullptr) Invalid("output_final_state=1 needs a final_state buffer");
    plan.params.out = out;
    plan.params.final_state = want_state ? final_state : nullptr;
    return plan.params;
}

}  // namespace xm

extern "C" {

void xm_gated_deltanet2_attrs_default(xm_gated_deltanet2_attrs_t *attrs) {
    if (attrs == nullptr) return;
    attrs->scale = 1.0f;                   // reference :47
    attrs->use_qk_l2norm_in_kernel = 1;    // reference :48
    attrs->output_final_state = 0;
    attrs->use_gate_in_kernel = 0;
    attrs->has_cu_seqlens = 0;
    attrs->state_v_first = 0;
}

int xm_gated_deltanet2_check_attrs(const xm_gated_deltanet2_attrs_t *attrs, char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::CheckAttrs(*attrs);
    });
}

int xm_gated_deltanet2_validate(const xm_tensor_t *inputs, size_t n_inputs, const xm_gated_deltanet2_attrs_t *attrs,
                                int64_t *out_shape, int32_t *out_rank, size_t *scratch_bytes, char *errbuf,
                                size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::CheckAttrs(*attrs);
        xm::Plan plan = xm::Prepare(inputs, n_inputs, *attrs);
        xm::WriteShape(plan.out_shape, out_shape, out_rank);
        if (scratch_bytes) *scratch_bytes = plan.scratch;
    });
}

int xm_gated_deltanet2_forward(const xm_tensor_t *inputs, size_t n_inputs, const xm_gated_deltanet2_attrs_t *attrs,
                               float *out, void *stream, const xm_allocator_t *alloc, char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        if (attrs->output_final_state != 0)
            xm::Invalid("GatedDeltaNet2Fn with output_final_state=1 needs a final_state output "
                        "(xm_gated_deltanet2_forward_states)");
        xm::Forward(inputs, n_inputs, *attrs, out, nullptr, stream, alloc);
    });
}

int xm_gated_deltanet2_forward_states(const xm_tensor_t *inputs, size_t n_inputs,
                                      const xm_gated_deltanet2_attrs_t *attrs, float *out, float *final_state,
                                      void *stream, const xm_allocator_t *alloc, char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::Forward(inputs, n_inputs, *attrs, out, final_state, stream, alloc);
    });
}

}  // extern "C"
