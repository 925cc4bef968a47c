// Mamba3SisoFn host layer: attribute checks, shape validation and launch.
// Mirrors mamba3_siso_fn_ort.cpp:43-227 of the reference (constructor checks
// in the same order, ValidateInputs and its messages, ToIntDim, output shape
// = V.shape) and the launcher's re-checks (mamba3_siso_fwd.cu:177-188).
// The fused kernel keeps the state in VGPRs, so headdim_qk is limited to 256
// (the reference's limit is its shared-memory budget, P*N + A + 4N + 128
// floats).  No scratch.
#include "xm_common.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr size_t kNumInputs = 11;

void CheckAttrs(const xm_mamba3_siso_attrs_t &a) {
    if (a.chunk_size <= 0) Invalid("Mamba3SisoFn requires chunk_size > 0");
    if (a.return_final_states != 0) Unsupported("Mamba3SisoFn v1 does not support return_final_states");
    if (a.has_input_states != 0) Unsupported("Mamba3SisoFn v1 does not support input states");
    if (a.has_cu_seqlens != 0) Unsupported("Mamba3SisoFn v1 does not support cu_seqlens");
}

struct Plan {
    Mamba3SisoParams params{};
    std::vector<int64_t> out_shape;
};

Plan Validate(const std::vector<View> &in, const xm_mamba3_siso_attrs_t &attrs) {
    const View &Q = in[0], &K = in[1], &V = in[2], &ADT = in[3], &DT = in[4], &Trap = in[5];
    const View &Qb = in[6], &Kb = in[7], &Ang = in[8], &D = in[9], &Z = in[10];
    // ValidateInputs (reference :146-227)
    RequireRank(Q, 4, "Q");
    RequireRank(K, 4, "K");
    RequireRank(V, 4, "V");
    RequireRank(ADT, 3, "ADT");
    RequireRank(DT, 3, "DT");
    RequireRank(Trap, 3, "Trap");
    RequireRank(Qb, 2, "Q_bias");
    RequireRank(Kb, 2, "K_bias");
    RequireRank(Ang, 4, "Angles");
    RequireSameShape(Q, K, "Q", "K");
    RequireSameShape(ADT, DT, "ADT", "DT");
    RequireSameShape(ADT, Trap, "ADT", "Trap");
    const int64_t batch = Q.shape[0], seqlen = Q.shape[1], nheads_qk = Q.shape[2], headdim_qk = Q.shape[3];
    const int64_t nheads = V.shape[2], headdim_v = V.shape[3], headdim_angles = Ang.shape[3];
    if (V.shape[0] != batch || V.shape[1] != seqlen) Invalid("V batch/seqlen must match Q");
    if (ADT.shape[0] != batch || ADT.shape[1] != nheads || ADT.shape[2] != seqlen)
        Invalid("ADT must have shape (batch, nheads, seqlen)");
    if (Qb.shape[0] != nheads || Qb.shape[1] != headdim_qk) Invalid("Q_bias must have shape (nheads, headdim_qk)");
    if (Kb.shape != Qb.shape) Invalid("K_bias shape must match Q_bias");
    if (Ang.shape[0] != batch || Ang.shape[1] != seqlen || Ang.shape[2] != nheads)
        Invalid("Angles must have shape (batch, seqlen, nheads, headdim_angles)");
    if (nheads_qk <= 0 || nheads <= 0 || nheads % nheads_qk != 0)
        Invalid("Mamba3SisoFn requires nheads divisible by nheads_qk");
    if (headdim_qk <= 0 || headdim_qk % 2 != 0) Invalid("Mamba3SisoFn requires positive even headdim_qk");
    if (headdim_v <= 0) Invalid("Mamba3SisoFn requires positive headdim_v");
    if (headdim_angles <= 0 || headdim_angles > headdim_qk / 2)
        Invalid("Mamba3SisoFn requires 0 < headdim_angles <= headdim_qk / 2");
    const bool has_d = D.present();
    const bool has_z = Z.present();
    if (has_d != (attrs.has_d != 0)) Invalid("Mamba3SisoFn has_d attribute does not match D input");
    if (has_z != (attrs.has_z != 0)) Invalid("Mamba3SisoFn has_z attribute does not match Z input");
    if (has_d) {
        RequireRank(D, 1, "D");
        if (D.shape[0] != nheads) Invalid("D must have shape (nheads,)");
    }
    if (has_z) {
        RequireRank(Z, 4, "Z");
        if (Z.shape[0] != batch || Z.shape[1] != seqlen || Z.shape[2] != nheads || Z.shape[3] != headdim_v)
            Invalid("Z must have shape (batch, seqlen, nheads, headdim_v)");
    }
    Plan plan;
    plan.out_shape = V.shape;
    Mamba3SisoParams &p = plan.params;
    p.batch = ToIntDim(Q.shape[0], "batch");
    p.seqlen = ToIntDim(Q.shape[1], "seqlen");
    p.nheads_qk = ToIntDim(Q.shape[2], "nheads_qk");
    p.n = ToIntDim(Q.shape[3], "headdim_qk");
    p.nheads = ToIntDim(V.shape[2], "nheads");
    p.p = ToIntDim(V.shape[3], "headdim_v");
    p.a = ToIntDim(Ang.shape[3], "headdim_angles");
    if (p.n > 256) Unsupported("Mamba3SisoFn supports headdim_qk up to 256");
    p.Q = Q.data;
    p.K = K.data;
    p.V = V.data;
    p.ADT = ADT.data;
    p.DT = DT.data;
    p.Trap = Trap.data;
    p.Q_bias = Qb.data;
    p.K_bias = Kb.data;
    p.Angles = Ang.data;
    p.D = has_d ? D.data : nullptr;
    p.Z = has_z ? Z.data : nullptr;
    return plan;
}

}  // namespace
}  // namespace xm

extern "C" {

void xm_mamba3_siso_attrs_default(xm_mamba3_siso_attrs_t *attrs) {
    if (attrs == nullptr) return;
    attrs->chunk_size = 64;   // reference :44
    attrs->has_d = 1;         // reference :45
    attrs->has_z = 1;         // reference :46
    attrs->return_final_states = 0;
    attrs->has_input_states = 0;
    attrs->has_cu_seqlens = 0;
}

int xm_mamba3_siso_check_attrs(const xm_mamba3_siso_attrs_t *attrs, char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::CheckAttrs(*attrs);
    });
}

int xm_mamba3_siso_validate(const xm_tensor_t *inputs, size_t n_inputs, const xm_mamba3_siso_attrs_t *attrs,
                            int64_t *out_shape, int32_t *out_rank, size_t *scratch_bytes, char *errbuf,
                            size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::CheckAttrs(*attrs);
        auto views = xm::MakeViews(inputs, n_inputs, xm::kNumInputs, "Mamba3SisoFn");
        xm::Plan plan = xm::Validate(views, *attrs);
        xm::WriteShape(plan.out_shape, out_shape, out_rank);
        if (scratch_bytes) *scratch_bytes = 0;
    });
}

int xm_mamba3_siso_forward(const xm_tensor_t *inputs, size_t n_inputs, const xm_mamba3_siso_attrs_t *attrs,
                           float *out, void *stream, const xm_allocator_t *alloc, char *errbuf, size_t errlen) {
    (void)alloc;
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        xm::CheckAttrs(*attrs);
        auto views = xm::MakeViews(inputs, n_inputs, xm::kNumInputs, "Mamba3SisoFn");
        xm::Plan plan = xm::Validate(views, *attrs);
        if (out == nullptr) xm::Invalid("output pointer is null");
        plan.params.out = out;
        xm::LaunchMamba3Siso(plan.params, stream);
    });
}

}  // extern "C"
