// Mamba3SisoFn host layer: attribute checks, shape validation and launch.
// Mirrors mamba3_siso_fn_ort.cpp:43-227 of the reference (constructor checks
// in the same order, ValidateInputs and its messages, ToIntDim, output shape
// = V.shape) and the launcher's re-checks (mamba3_siso_fwd.cu:177-188).
// The kernels keep the state in VGPRs and a block of rotated q/k rows in LDS:
// up to 512 keys in one launch (32 keys per lane of a 16-lane row, 16-token
// blocks: 155 KiB of LDS), above that one launch per block of 512 keys, each
// adding its part of the output.  The reference's limit is its shared-memory
// budget of P*N + A + 4N + 128 floats (mamba3_siso_fwd.cu:190-207), e.g.
// N = 576 at P = 64 or about 2000 at P = 16 on a 160 KiB device; this layer
// takes any even headdim_qk.  N up to 256 takes the chunked fp32-MFMA kernel,
// above that the token-by-token kernel.  No scratch.
//
// Widening: has_input_states = 1 and return_final_states = 1, which the
// reference rejects (:50-55), are accepted.  The states are (ssm [B,H,P,N],
// angle [B,H,A], k [B,H,N], v [B,H,P]): S and the angle state after the last
// token, that token's rotated k and its V.  Input states come as inputs
// 11-14 (15 inputs); final states go to the four buffers of
// xm_mamba3_siso_forward_states.  Two calls chained through the states give
// the outputs and states of one call.
// Widening: has_cu_seqlens = 1 (rejected at :56-58) packs N sequences along
// seqlen: input 15 is cu_seqlens (int64 [N+1]; 16 inputs, of which 11-14, the
// states, are empty unless has_input_states = 1), the tensors have batch 1
// and the states are [N, ...]; the kernel reads each sequence's token range
// on the device.
#include "xm_common.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr size_t kNumInputs = 11;
constexpr size_t kNumInputsWithStates = 15;
constexpr size_t kNumInputsPacked = 16;   // cu_seqlens at 15, the state slots 11-14 before it

void CheckAttrs(const xm_mamba3_siso_attrs_t &a) {
    if (a.chunk_size <= 0) Invalid("Mamba3SisoFn requires chunk_size > 0");
}

size_t ExpectedInputs(const xm_mamba3_siso_attrs_t &a) {
    if (a.has_cu_seqlens != 0) return kNumInputsPacked;
    return a.has_input_states != 0 ? kNumInputsWithStates : kNumInputs;
}

struct Plan {
    Mamba3SisoParams params{};
    std::vector<int64_t> out_shape;
};

Plan Validate(const std::vector<View> &in, const IndexView *cu, const xm_mamba3_siso_attrs_t &attrs) {
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
    // packed sequences: one row of tokens, one state per sequence
    if (cu != nullptr && batch != 1)
        Invalid("Mamba3SisoFn with cu_seqlens requires batch 1 (sequences packed along seqlen)");
    const int64_t nstate = cu != nullptr ? cu->count - 1 : batch;
    Plan plan;
    plan.out_shape = V.shape;
    Mamba3SisoParams &p = plan.params;
    p.batch = ToIntDim(nstate, cu != nullptr ? "sequences" : "batch");
    p.cu_seqlens = cu != nullptr ? cu->data : nullptr;
    p.seqlen = ToIntDim(Q.shape[1], "seqlen");
    p.nheads_qk = ToIntDim(Q.shape[2], "nheads_qk");
    p.n = ToIntDim(Q.shape[3], "headdim_qk");
    p.nheads = ToIntDim(V.shape[2], "nheads");
    p.p = ToIntDim(V.shape[3], "headdim_v");
    p.a = ToIntDim(Ang.shape[3], "headdim_angles");
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
    if (attrs.has_input_states == 0) {
        for (size_t i = kNumInputs; i < in.size(); ++i)
            if (in[i].present()) Invalid("Mamba3SisoFn state inputs need has_input_states=1");
    } else {
        const View &Ss = in[11], &As = in[12], &Ks = in[13], &Vs = in[14];
        RequireRank(Ss, 4, "ssm_state");
        RequireRank(As, 3, "angle_state");
        RequireRank(Ks, 3, "k_state");
        RequireRank(Vs, 3, "v_state");
        if (Ss.shape != std::vector<int64_t>{nstate, nheads, headdim_v, headdim_qk})
            Invalid("ssm_state must have shape (batch, nheads, headdim_v, headdim_qk)");
        if (As.shape != std::vector<int64_t>{nstate, nheads, headdim_angles})
            Invalid("angle_state must have shape (batch, nheads, headdim_angles)");
        if (Ks.shape != std::vector<int64_t>{nstate, nheads, headdim_qk})
            Invalid("k_state must have shape (batch, nheads, headdim_qk)");
        if (Vs.shape != std::vector<int64_t>{nstate, nheads, headdim_v})
            Invalid("v_state must have shape (batch, nheads, headdim_v)");
        p.in_ssm = Ss.data;
        p.in_angle = As.data;
        p.in_k = Ks.data;
        p.in_v = Vs.data;
    }
    return plan;
}

// The float views (and cu_seqlens, the last input, when packed) and the plan.
Plan Prepare(const xm_tensor_t *inputs, size_t n_inputs, const xm_mamba3_siso_attrs_t &attrs) {
    const size_t expected = ExpectedInputs(attrs);
    const bool packed = attrs.has_cu_seqlens != 0;
    auto views = MakeViews(inputs, n_inputs, expected, "Mamba3SisoFn", packed ? kNumInputsWithStates : expected);
    if (!packed) return Validate(views, nullptr, attrs);
    const IndexView cu = MakeIndexView(inputs[kNumInputsWithStates], "cu_seqlens");
    return Validate(views, &cu, attrs);
}

void Forward(const xm_tensor_t *inputs, size_t n_inputs, const xm_mamba3_siso_attrs_t &attrs, float *out,
             float *const *states, void *stream) {
    ResetLaunches();
    CheckAttrs(attrs);
    Plan plan = Prepare(inputs, n_inputs, attrs);
    if (out == nullptr) Invalid("output pointer is null");
    plan.params.out = out;
    if (attrs.return_final_states != 0) {
        for (int i = 0; i < 4; ++i)
            if (states == nullptr || states[i] == nullptr) Invalid("return_final_states=1 needs four state buffers");
        plan.params.f_ssm = states[0];
        plan.params.f_angle = states[1];
        plan.params.f_k = states[2];
        plan.params.f_v = states[3];
    }
    LaunchMamba3Siso(plan.params, stream);
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
        xm::Plan plan = xm::Prepare(inputs, n_inputs, *attrs);
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
        if (attrs->return_final_states != 0)
            xm::Invalid("Mamba3SisoFn with return_final_states=1 needs final-state outputs "
                        "(xm_mamba3_siso_forward_states)");
        xm::Forward(inputs, n_inputs, *attrs, out, nullptr, stream);
    });
}

int xm_mamba3_siso_forward_states(const xm_tensor_t *inputs, size_t n_inputs, const xm_mamba3_siso_attrs_t *attrs,
                                  float *out, float *ssm_state, float *angle_state, float *k_state, float *v_state,
                                  void *stream, const xm_allocator_t *alloc, char *errbuf, size_t errlen) {
    (void)alloc;
    return xm::Guard(errbuf, errlen, [&] {
        if (attrs == nullptr) xm::Invalid("attrs is null");
        float *const states[4] = {ssm_state, angle_state, k_state, v_state};
        xm::Forward(inputs, n_inputs, *attrs, out, states, stream);
    });
}

}  // extern "C"
