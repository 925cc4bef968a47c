// Test double of the two pieces of ONNX Runtime's C++ wrapper that the
// custom-op layer uses: Ort::InitApi (ORT_API_MANUAL_INIT) and the
// Ort::CustomOpBase<TOp, TKernel> helper, which fills the OrtCustomOp table
// with calls into the operator class TOp and its kernel class TKernel, with
// REQUIRED inputs/outputs unless TOp says otherwise.  Test infrastructure only.
#ifndef XM_TEST_ORT_DOUBLE_CXX_API_H_
#define XM_TEST_ORT_DOUBLE_CXX_API_H_

#include "onnxruntime_c_api.h"

namespace Ort {

namespace detail {
inline const OrtApi *&ApiSlot() {
    static const OrtApi *api = nullptr;
    return api;
}
}  // namespace detail

inline void InitApi(const OrtApi *api) noexcept { detail::ApiSlot() = api; }
inline const OrtApi &GetApi() noexcept { return *detail::ApiSlot(); }

template <typename TOp, typename TKernel>
struct CustomOpBase : OrtCustomOp {
    CustomOpBase() {
        OrtCustomOp::version = ORT_API_VERSION;
        OrtCustomOp::CreateKernel = [](const OrtCustomOp *self, const OrtApi *api, const OrtKernelInfo *info) -> void * {
            return static_cast<const TOp *>(self)->CreateKernel(*api, info);
        };
        OrtCustomOp::GetName = [](const OrtCustomOp *self) { return static_cast<const TOp *>(self)->GetName(); };
        OrtCustomOp::GetExecutionProviderType = [](const OrtCustomOp *self) {
            return static_cast<const TOp *>(self)->GetExecutionProviderType();
        };
        OrtCustomOp::GetInputTypeCount = [](const OrtCustomOp *self) {
            return static_cast<const TOp *>(self)->GetInputTypeCount();
        };
        OrtCustomOp::GetInputType = [](const OrtCustomOp *self, size_t i) {
            return static_cast<const TOp *>(self)->GetInputType(i);
        };
        OrtCustomOp::GetOutputTypeCount = [](const OrtCustomOp *self) {
            return static_cast<const TOp *>(self)->GetOutputTypeCount();
        };
        OrtCustomOp::GetOutputType = [](const OrtCustomOp *self, size_t i) {
            return static_cast<const TOp *>(self)->GetOutputType(i);
        };
        OrtCustomOp::KernelCompute = [](void *kernel, OrtKernelContext *ctx) {
            static_cast<TKernel *>(kernel)->Compute(ctx);
        };
        OrtCustomOp::KernelDestroy = [](void *kernel) { delete static_cast<TKernel *>(kernel); };
        OrtCustomOp::GetInputCharacteristic = [](const OrtCustomOp *self, size_t i) {
            return static_cast<const TOp *>(self)->GetInputCharacteristic(i);
        };
        OrtCustomOp::GetOutputCharacteristic = [](const OrtCustomOp *self, size_t i) {
            return static_cast<const TOp *>(self)->GetOutputCharacteristic(i);
        };
    }
    const char *GetExecutionProviderType() const { return nullptr; }
    OrtCustomOpInputOutputCharacteristic GetInputCharacteristic(size_t) const { return INPUT_OUTPUT_REQUIRED; }
    OrtCustomOpInputOutputCharacteristic GetOutputCharacteristic(size_t) const { return INPUT_OUTPUT_REQUIRED; }
};

}  // namespace Ort

#endif  // XM_TEST_ORT_DOUBLE_CXX_API_H_
