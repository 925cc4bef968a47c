// SelectiveScanFn host layer: attribute checks, shape validation and launch.
//
// Mirrors the reference adapter selective_scan_fn_ort.cpp:50-197 (constructor
// checks, MaybeInsertGroupDim, the Compute validation and its messages).
// d_state = 0 is accepted as in the reference (its state loop is empty,
// selective_scan_fwd_kernel.cuh:161,166): y = D * u, or zeros without D.
// Differences, all on inputs the reference leaves unchecked and would read out
// of bounds or with mismatched strides:
//   - B/C/D/z/delta_bias extents must equal the extents the kernel reads;
//   - rank > 4 for B/C and n_groups < 1 are rejected;
//   - an empty u (any dimension 0) yields an empty output with no launch;
//   - no uint32 stride limit (the kernels index with 64-bit bases).
// No scratch is needed: the reference's per-chunk state buffer `x` is written
// and never read, and its gated `out_z` buffer is discarded (kernel.cuh:256,
// :296-299), so this implementation computes neither.
//
// Widening: return_last_state = 1, which the reference rejects (:52-55), is
// accepted through xm_selective_scan_forward_states, which also writes the
// scan state after the last token, [batch, dim, dstate] (the `last_state` of
// the Mamba selective_scan_fn interface).
// Widening: u, delta, z and variable B/C may be float16 or bfloat16 (one type
// for all), as in the reference's half / bfloat16 kernel instantiations that
// its fp32-only host cannot reach (ort_common.h:90-92); weights stay fp32 and
// y takes u's type.
#include "xm_common.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr size_t kNumInputs = 8;

void CheckAttrs(const xm_selective_scan_attrs_t &) {}

void RequireStateEntry(const xm_selective_scan_attrs_t &a) {
    if (a.return_last_state != 0)
        Invalid("SelectiveScanFn with return_last_state=1 needs a last_state output "
                "(xm_selective_scan_forward_states)");
}

// rearrange(B, "b dstate l -> b 1 dstate l") when rank 3 (reference :26-31, :77-78).
void MaybeInsertGroupDim(View &v) {
    if (v.rank() == 3) v.shape.insert(v.shape.begin() + 1, 1);
}

struct Plan {
    SelectiveScanParams params{};
    std::vector<int64_t> out_shape;
    bool empty = false;
};

Plan Validate(const std::vector<View> &in, const xm_selective_scan_attrs_t &attrs) {
    View u = in[0], delta = in[1], A = in[2], B = in[3], C = in[4], D = in[5], z = in[6], bias = in[7];
    MaybeInsertGroupDim(B);
    MaybeInsertGroupDim(C);
    if (u.rank() != 3) Invalid("u must be 3-D");
    if (delta.shape != u.shape) Invalid("delta must have same shape as u");
    if (A.rank() != 2) Invalid("A must be 2-D");
    if (B.rank() < 2) Invalid("B must have rank >= 2");
    if (C.rank() < 2) Invalid("C must have rank >= 2");
    if (B.rank() > 4) Invalid("B must have rank <= 4");
    if (C.rank() > 4) Invalid("C must have rank <= 4");

    const int64_t batch = u.shape[0], dim = u.shape[1], seqlen = u.shape[2];
    const int64_t dstate = A.shape[1];
    if (A.shape[0] != dim) Invalid("A dimension mismatch with u");
    if (dstate > 256) Invalid("selective_scan supports d_state up to 256");
    if (batch > INT32_MAX || dim > INT32_MAX || seqlen > INT32_MAX) Invalid("u dimension is out of range");

    const bool b_var = B.rank() >= 3;
    const bool c_var = C.rank() >= 3;
    const int64_t n_groups = b_var ? B.shape[1] : 1;
    if (n_groups < 1) Invalid("n_groups must be positive");
    if (dim % n_groups != 0) Invalid("dim must be divisible by n_groups");

    // Extents the kernel reads (unchecked by the reference).
    if (b_var) {
        if (B.shape[0] != batch || B.shape[2] != dstate || B.shape[3] != seqlen)
            Invalid("B must have shape (batch, n_groups, dstate, seqlen) when variable");
    } else if (B.shape[0] != dim || B.shape[1] != dstate) {
        Invalid("B must have shape (dim, dstate) when constant");
    }
    int64_t groups_c = 1;
    if (c_var) {
        groups_c = C.shape[1];
        // Channel d reads C group d / (dim / n_groups) when B is variable and
        // group 0 when B is constant (n_groups comes from B, reference :109).
        if (C.shape[0] != batch || C.shape[2] != dstate || C.shape[3] != seqlen || groups_c < (b_var ? n_groups : 1))
            Invalid("C must have shape (batch, n_groups, dstate, seqlen) when variable");
    } else if (C.shape[0] != dim || C.shape[1] != dstate) {
        Invalid("C must have shape (dim, dstate) when constant");
    }
    if (D.present() && !(D.rank() == 1 && D.shape[0] == dim)) Invalid("D must have shape (dim,)");
    if (z.present() && z.shape != u.shape) Invalid("z must have same shape as u");
    if (bias.present() && !(bias.rank() == 1 && bias.shape[0] == dim)) Invalid("delta_bias must have shape (dim,)");
    // element types: the data tensors share u's; the weights are fp32
    const int32_t et = u.elem;
    const bool types_ok = delta.elem == et && (!z.present() || z.elem == et) &&
                          (b_var ? B.elem == et : B.elem == XM_ELEM_FLOAT) &&
                          (c_var ? C.elem == et : C.elem == XM_ELEM_FLOAT);
    if (!types_ok)
        Invalid("SelectiveScanFn: u, delta, z and variable B/C must share one element type; "
                "constant B/C are float32");

    Plan plan;
    plan.out_shape = u.shape;
    plan.empty = batch == 0 || dim == 0 || seqlen == 0;
    SelectiveScanParams &p = plan.params;
    p.u = u.data;
    p.delta = delta.data;
    p.A = A.data;
    p.B = B.data;
    p.C = C.data;
    p.D = D.present() ? D.data : nullptr;
    p.delta_bias = bias.present() ? bias.data : nullptr;
    p.out = nullptr;
    p.batch = static_cast<int>(batch);
    p.dim = static_cast<int>(dim);
    p.seqlen = static_cast<int>(seqlen);
    p.dstate = static_cast<int>(dstate);
    p.b_var = b_var;
    p.c_var = c_var;
    p.groups_b = static_cast<int>(n_groups);
    p.groups_c = static_cast<int>(groups_c);
    p.dim_per_group = static_cast<int>(dim / n_groups);
    p.delta_softplus = attrs.delta_softplus != 0;
    p.in_type = et;
    return plan;
}

// Views of the eight inputs: u, delta, B, C and z may be 16-bit.
std::vector<View> SsViews(const xm_tensor_t *inputs, size_t n_inputs) {
    if (inputs == nullptr) Invalid("SelectiveScanFn received a null input array");
    if (n_inputs != kNumInputs)
        Invalid("SelectiveScanFn expects " + std::to_string(kNumInputs) + " inputs, got " + std::to_string(n_inputs));
    std::vector<View> v;
    for (size_t i = 0; i < kNumInputs; ++i) v.push_back(MakeView(inputs[i], i <= 1 || i == 3 || i == 4 || i == 6));
    return v;
}

void Forward(const xm_tensor_t *inputs, size_t n_inputs, const xm_selective_scan_attrs_t &attrs, void *out,
             float *last_state, void *stream) {
    ResetLaunches();
    CheckAttrs(attrs);
    auto views = SsViews(inputs, n_inputs);
    Plan plan = Validate(views, attrs);
    const bool want_state = attrs.return_last_state != 0;
    if (want_state && last_state == nullptr) Invalid("return_last_state=1 needs a last_state buffer");
    plan.params.last_state = want_state ? last_state : nullptr;
    if (plan.empty) {
        // no tokens: the state is the zero initial state
        const size_t state_elems = static_cast<size_t>(plan.params.batch) * plan.params.dim * plan.params.dstate;
        if (want_state) LaunchFillZeros(last_state, state_elems, stream);
        return;
    }
    if (out == nullptr) Invalid("output pointer is null");
    plan.params.out = out;
    LaunchSelectiveScan(plan.params, stream);
}

}  // namespace
}  // namespace xm

extern "C" {

void xm_selective_scan_attrs_default(xm_selective_scan_attrs_t *attrs) {
    if (attrs == nullptr) return;
    attrs->delta_softplus = 0;     // reference :51
    attrs->return_last_state = 0;  // reference :52
}

int xm_selective_scan_check_attrs(const xm_selective_scan_attrs_t *attrs, char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::CheckAttrs(*attrs);
    });
}

int xm_selective_scan_validate(const xm_tensor_t *inputs, size_t n_inputs, const xm_selective_scan_attrs_t *attrs,
                               int64_t *out_shape, int32_t *out_rank, size_t *scratch_bytes, char *errbuf,
                               size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::CheckAttrs(*attrs);
        auto views = xm::SsViews(inputs, n_inputs);
        xm::Plan plan = xm::Validate(views, *attrs);
        xm::WriteShape(plan.out_shape, out_shape, out_rank);
        if (scratch_bytes) *scratch_bytes = 0;
    });
}

int xm_selective_scan_forward(const xm_tensor_t *inputs, size_t n_inputs, const xm_selective_scan_attrs_t *attrs,
                              void *out, void *stream, const xm_allocator_t *alloc, char *errbuf, size_t errlen) {
    (void)alloc;
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::RequireStateEntry(*attrs);
        xm::Forward(inputs, n_inputs, *attrs, out, nullptr, stream);
    });
}

int xm_selective_scan_forward_states(const xm_tensor_t *inputs, size_t n_inputs,
                                     const xm_selective_scan_attrs_t *attrs, void *out, float *last_state,
                                     void *stream, const xm_allocator_t *alloc, char *errbuf, size_t errlen) {
    (void)alloc;
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::Forward(inputs, n_inputs, *attrs, out, last_state, stream);
    });
}

}  // extern "C"
