// ONNX Runtime descriptors and kernels of the three device operators.
//
// Names, input counts, element types and attribute names/defaults are the
// reference's (selective_scan_fn_ort.cpp:48-56, :235-246;
// mamba3_siso_fn_ort.cpp:41-59, :235-246; gated_deltanet2_fn_ort.cpp:44-64,
// :226-237); the execution provider is ROCm.  Attribute checks run in the
// kernel constructor (session creation), shape checks in Compute (Run), both
// through the C ABI, which carries the reference's messages.
//
// Widening: SelectiveScanFn with return_last_state=1 and GatedDeltaNet2Fn
// with output_final_state=1, which the reference rejects, fill an optional
// output 1 with the state after the last token ([B,D,N] and [B,H,K,V]).
// Mamba3SisoFn with return_final_states=1 fills optional outputs 1-4 (ssm
// [B,H,P,N], angle [B,H,A], k [B,H,N], v [B,H,P]) and with has_input_states=1
// takes the same four as optional inputs 11-14.
// Widening: SelectiveScanFn is also registered for float16 and bfloat16
// data (u, delta, variable B/C, z and y; A, D, delta_bias and the state
// stay float), the reference's half / bfloat16 kernel instantiations, which
// its fp32-only host cannot reach.  ONNX Runtime picks the descriptor by the
// node's input types; constant B/C with 16-bit data is a C ABI case only.
// Widening: has_cu_seqlens=1 (GatedDeltaNet2Fn, Mamba3SisoFn) takes the
// packed sequences' offsets as an optional int64 input (7 and 15); the
// states then have one row per sequence.
#include "ort_glue.h"

namespace {

using xm_ort::Check;
using xm_ort::ComputeDeviceOp;
using xm_ort::FloatAttr;
using xm_ort::IntAttr;
using xm_ort::StateOutputs;


// ---- SelectiveScanFn -------------------------------------------------------
class SelectiveScanKernel {
public:
    SelectiveScanKernel(const OrtApi &api, const OrtKernelInfo *info) : api_(api) {
        xm_selective_scan_attrs_default(&attrs_);
        attrs_.delta_softplus = IntAttr(api, info, "delta_softplus", attrs_.delta_softplus);
        attrs_.return_last_state = IntAttr(api, info, "return_last_state", attrs_.return_last_state);
        char err[512];
        Check(xm_selective_scan_check_attrs(&attrs_, err, sizeof(err)), err);
    }
    void Compute(OrtKernelContext *ctx) {
        const bool want = attrs_.return_last_state != 0;
        auto state = [want](const xm_tensor_t *in) {
            StateOutputs so;
            so.what = "return_last_state";
            if (want) {   // [B, D, N]: u is [B, D, L] and A is [D, N] (validated)
                so.count = 1;
                so.rank[0] = 3;
                so.shape[0][0] = in[0].shape[0];
                so.shape[0][1] = in[0].shape[1];
                so.shape[0][2] = in[2].shape[1];
            }
            return so;
        };
        auto launch = [](const xm_tensor_t *in, size_t n, const xm_selective_scan_attrs_t *a, void *out,
                         float *const *states, void *stream, const xm_allocator_t *alloc, char *err, size_t errlen) {
            return xm_selective_scan_forward_states(in, n, a, out, states[0], stream, alloc, err, errlen);
        };
        ComputeDeviceOp(api_, ctx, 8, 8, attrs_, xm_selective_scan_validate, state, launch);
    }

private:
    const OrtApi &api_;
    xm_selective_scan_attrs_t attrs_{};
};

// DT: the element type of the data tensors (inputs 0, 1, 3, 4, 6 and output 0).
template <ONNXTensorElementDataType DT>
struct SelectiveScanOpT : Ort::CustomOpBase<SelectiveScanOpT<DT>, SelectiveScanKernel> {
    void *CreateKernel(const OrtApi &api, const OrtKernelInfo *info) const { return new SelectiveScanKernel(api, info); }
    const char *GetName() const { return "SelectiveScanFn"; }
    const char *GetExecutionProviderType() const { return XM_ORT_GPU_EP; }
    size_t GetInputTypeCount() const { return 8; }
    ONNXTensorElementDataType GetInputType(size_t i) const {
        return (i <= 1 || i == 3 || i == 4 || i == 6) ? DT : ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT;
    }
    size_t GetOutputTypeCount() const { return 2; }
    ONNXTensorElementDataType GetOutputType(size_t i) const { return i == 0 ? DT : ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT; }
    OrtCustomOpInputOutputCharacteristic GetOutputCharacteristic(size_t i) const {
        return i == 0 ? INPUT_OUTPUT_REQUIRED : INPUT_OUTPUT_OPTIONAL;
    }
};
using SelectiveScanOp = SelectiveScanOpT<ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT>;

// ---- Mamba3SisoFn ----------------------------------------------------------
class Mamba3SisoKernel {
public:
    Mamba3SisoKernel(const OrtApi &api, const OrtKernelInfo *info) : api_(api) {
        xm_mamba3_siso_attrs_default(&attrs_);
        attrs_.chunk_size = IntAttr(api, info, "chunk_size", attrs_.chunk_size);
        attrs_.has_d = IntAttr(api, info, "has_d", attrs_.has_d);
        attrs_.has_z = IntAttr(api, info, "has_z", attrs_.has_z);
        attrs_.return_final_states = IntAttr(api, info, "return_final_states", attrs_.return_final_states);
        attrs_.has_input_states = IntAttr(api, info, "has_input_states", attrs_.has_input_states);
        attrs_.has_cu_seqlens = IntAttr(api, info, "has_cu_seqlens", attrs_.has_cu_seqlens);
        char err[512];
        Check(xm_mamba3_siso_check_attrs(&attrs_, err, sizeof(err)), err);
    }
    void Compute(OrtKernelContext *ctx) {
        const bool want = attrs_.return_final_states != 0, packed = attrs_.has_cu_seqlens != 0;
        auto state = [want, packed](const xm_tensor_t *in) {
            StateOutputs so;
            so.what = "return_final_states";
            if (want) {   // Q [B,T,Hq,N], V [B,T,H,P], Angles [B,T,H,A], cu_seqlens [N+1] (validated)
                const int64_t b = packed ? in[15].shape[0] - 1 : in[0].shape[0];
                const int64_t n = in[0].shape[3], h = in[2].shape[2], p = in[2].shape[3];
                const int64_t a = in[8].shape[3];
                const int64_t shapes[4][4] = {{b, h, p, n}, {b, h, a, 0}, {b, h, n, 0}, {b, h, p, 0}};
                so.count = 4;
                for (int i = 0; i < 4; ++i) {
                    so.rank[i] = i == 0 ? 4 : 3;
                    for (int d = 0; d < so.rank[i]; ++d) so.shape[i][d] = shapes[i][d];
                }
            }
            return so;
        };
        auto launch = [](const xm_tensor_t *in, size_t n, const xm_mamba3_siso_attrs_t *a, void *out,
                         float *const *states, void *stream, const xm_allocator_t *alloc, char *err, size_t errlen) {
            return xm_mamba3_siso_forward_states(in, n, a, static_cast<float *>(out), states[0], states[1], states[2], states[3], stream,
                                                 alloc, err, errlen);
        };
        ComputeDeviceOp(api_, ctx, 11, 16, attrs_, xm_mamba3_siso_validate, state, launch);
    }

private:
    const OrtApi &api_;
    xm_mamba3_siso_attrs_t attrs_{};
};

struct Mamba3SisoOp : Ort::CustomOpBase<Mamba3SisoOp, Mamba3SisoKernel> {
    void *CreateKernel(const OrtApi &api, const OrtKernelInfo *info) const { return new Mamba3SisoKernel(api, info); }
    const char *GetName() const { return "Mamba3SisoFn"; }
    const char *GetExecutionProviderType() const { return XM_ORT_GPU_EP; }
    size_t GetInputTypeCount() const { return 16; }
    ONNXTensorElementDataType GetInputType(size_t i) const {
        return i == 15 ? ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64 : ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT;   // cu_seqlens
    }
    OrtCustomOpInputOutputCharacteristic GetInputCharacteristic(size_t i) const {
        return i < 11 ? INPUT_OUTPUT_REQUIRED : INPUT_OUTPUT_OPTIONAL;
    }
    size_t GetOutputTypeCount() const { return 5; }
    ONNXTensorElementDataType GetOutputType(size_t) const { return ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT; }
    OrtCustomOpInputOutputCharacteristic GetOutputCharacteristic(size_t i) const {
        return i == 0 ? INPUT_OUTPUT_REQUIRED : INPUT_OUTPUT_OPTIONAL;
    }
};

// ---- GatedDeltaNet2Fn ------------------------------------------------------
class GatedDeltaNet2Kernel {
public:
    GatedDeltaNet2Kernel(const OrtApi &api, const OrtKernelInfo *info) : api_(api) {
        xm_gated_deltanet2_attrs_default(&attrs_);
        attrs_.scale = FloatAttr(api, info, "scale", attrs_.scale);
        attrs_.use_qk_l2norm_in_kernel = IntAttr(api, info, "use_qk_l2norm_in_kernel", attrs_.use_qk_l2norm_in_kernel);
        attrs_.output_final_state = IntAttr(api, info, "output_final_state", attrs_.output_final_state);
        attrs_.use_gate_in_kernel = IntAttr(api, info, "use_gate_in_kernel", attrs_.use_gate_in_kernel);
        attrs_.has_cu_seqlens = IntAttr(api, info, "has_cu_seqlens", attrs_.has_cu_seqlens);
        attrs_.state_v_first = IntAttr(api, info, "state_v_first", attrs_.state_v_first);
        char err[512];
        Check(xm_gated_deltanet2_check_attrs(&attrs_, err, sizeof(err)), err);
    }
    void Compute(OrtKernelContext *ctx) {
        const bool want = attrs_.output_final_state != 0, packed = attrs_.has_cu_seqlens != 0;
        auto state = [want, packed](const xm_tensor_t *in) {
            StateOutputs so;
            so.what = "output_final_state";
            if (want) {   // [B, H, K, V]: q is [B, T, H, K], v is [B, T, H, V], cu_seqlens [B+1] (validated)
                so.count = 1;
                so.rank[0] = 4;
                so.shape[0][0] = packed ? in[7].shape[0] - 1 : in[0].shape[0];
                so.shape[0][1] = in[0].shape[2];
                so.shape[0][2] = in[0].shape[3];
                so.shape[0][3] = in[2].shape[3];
            }
            return so;
        };
        auto launch = [](const xm_tensor_t *in, size_t n, const xm_gated_deltanet2_attrs_t *a, void *out,
                         float *const *states, void *stream, const xm_allocator_t *alloc, char *err, size_t errlen) {
            return xm_gated_deltanet2_forward_states(in, n, a, static_cast<float *>(out), states[0], stream, alloc, err, errlen);
        };
        ComputeDeviceOp(api_, ctx, 7, 8, attrs_, xm_gated_deltanet2_validate, state, launch);
    }

private:
    const OrtApi &api_;
    xm_gated_deltanet2_attrs_t attrs_{};
};

struct GatedDeltaNet2Op : Ort::CustomOpBase<GatedDeltaNet2Op, GatedDeltaNet2Kernel> {
    void *CreateKernel(const OrtApi &api, const OrtKernelInfo *info) const { return new GatedDeltaNet2Kernel(api, info); }
    const char *GetName() const { return "GatedDeltaNet2Fn"; }
    const char *GetExecutionProviderType() const { return XM_ORT_GPU_EP; }
    size_t GetInputTypeCount() const { return 8; }
    ONNXTensorElementDataType GetInputType(size_t i) const {
        return i == 7 ? ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64 : ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT;   // cu_seqlens
    }
    OrtCustomOpInputOutputCharacteristic GetInputCharacteristic(size_t i) const {
        return i < 7 ? INPUT_OUTPUT_REQUIRED : INPUT_OUTPUT_OPTIONAL;
    }
    size_t GetOutputTypeCount() const { return 2; }
    ONNXTensorElementDataType GetOutputType(size_t) const { return ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT; }
    OrtCustomOpInputOutputCharacteristic GetOutputCharacteristic(size_t i) const {
        return i == 0 ? INPUT_OUTPUT_REQUIRED : INPUT_OUTPUT_OPTIONAL;
    }
};

// Descriptors live for the whole process: the domain that references them is
// never released.
SelectiveScanOp g_selective_scan_op;
SelectiveScanOpT<ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16> g_selective_scan_op_f16;
SelectiveScanOpT<ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16> g_selective_scan_op_bf16;
Mamba3SisoOp g_mamba3_siso_op;
GatedDeltaNet2Op g_gated_deltanet2_op;

}  // namespace

OrtStatus *XmAddSelectiveScanFnOp(const OrtApi &api, OrtCustomOpDomain *domain) {
    OrtStatus *st = api.CustomOpDomain_Add(domain, &g_selective_scan_op);
    if (st == nullptr) st = api.CustomOpDomain_Add(domain, &g_selective_scan_op_f16);
    if (st == nullptr) st = api.CustomOpDomain_Add(domain, &g_selective_scan_op_bf16);
    return st;
}
OrtStatus *XmAddMamba3SisoFnOp(const OrtApi &api, OrtCustomOpDomain *domain) {
    return api.CustomOpDomain_Add(domain, &g_mamba3_siso_op);
}
OrtStatus *XmAddGatedDeltaNet2FnOp(const OrtApi &api, OrtCustomOpDomain *domain) {
    return api.CustomOpDomain_Add(domain, &g_gated_deltanet2_op);
}
