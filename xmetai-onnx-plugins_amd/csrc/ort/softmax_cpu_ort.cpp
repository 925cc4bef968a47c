// SoftmaxCPU descriptor and kernel (CPU execution provider).  Reference:
// csrc/softmax_cpu/softmax_cpu_ort.cpp:20-114: one float input, one float
// output of the same shape, attribute "axis" (int, default -1).  The output
// is requested before the axis is checked, as in the reference, so an empty
// input succeeds whatever the axis.
#include "ort_glue.h"

namespace {

using xm_ort::Check;
using xm_ort::IntAttr;
using xm_ort::ThrowIfFailed;

class SoftmaxCpuKernel {
public:
    SoftmaxCpuKernel(const OrtApi &api, const OrtKernelInfo *info) : api_(api) {
        axis_ = IntAttr(api, info, "axis", -1);
    }
    void Compute(OrtKernelContext *ctx) {
        const OrtValue *in = nullptr;
        ThrowIfFailed(api_, api_.KernelContext_GetInput(ctx, 0, &in));
        const xm_tensor_t d = xm_ort::Describe(api_, in);
        if (d.elem_type != XM_ELEM_FLOAT) throw std::runtime_error("TensorView expects float32 tensors");
        OrtValue *out = nullptr;
        ThrowIfFailed(api_, api_.KernelContext_GetOutput(ctx, 0, d.shape, static_cast<size_t>(d.rank), &out));
        void *out_data = nullptr;
        ThrowIfFailed(api_, api_.GetTensorMutableData(out, &out_data));
        char err[256];
        Check(xm_softmax_cpu(static_cast<const float *>(d.data), d.shape, d.rank, axis_,
                             static_cast<float *>(out_data), err, sizeof(err)),
              err);
    }

private:
    const OrtApi &api_;
    int64_t axis_ = -1;
};

struct SoftmaxCpuOp : Ort::CustomOpBase<SoftmaxCpuOp, SoftmaxCpuKernel> {
    void *CreateKernel(const OrtApi &api, const OrtKernelInfo *info) const { return new SoftmaxCpuKernel(api, info); }
    const char *GetName() const { return "SoftmaxCPU"; }
    const char *GetExecutionProviderType() const { return "CPUExecutionProvider"; }
    size_t GetInputTypeCount() const { return 1; }
    ONNXTensorElementDataType GetInputType(size_t) const { return ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT; }
    size_t GetOutputTypeCount() const { return 1; }
    ONNXTensorElementDataType GetOutputType(size_t) const { return ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT; }
};

SoftmaxCpuOp g_softmax_cpu_op;

}  // namespace

OrtStatus *XmAddSoftmaxCpuOp(const OrtApi &api, OrtCustomOpDomain *domain) {
    return api.CustomOpDomain_Add(domain, &g_softmax_cpu_op);
}
