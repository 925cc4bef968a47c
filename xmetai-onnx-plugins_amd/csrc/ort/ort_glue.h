// Shared pieces of the ONNX Runtime custom-op layer: OrtValue -> xm_tensor_t
// descriptors, attribute reads with defaults, the scratch allocator adapter
// and the Compute skeleton every device operator uses.  The C++ wrapper header
// is used with ORT_API_MANUAL_INIT: RegisterCustomOps installs the OrtApi it
// receives, so the library has no link-time dependency on onnxruntime.
#pragma once

#ifndef ORT_API_MANUAL_INIT
#define ORT_API_MANUAL_INIT
#endif
#include <onnxruntime_cxx_api.h>

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "xmetai_recurrent.h"

#ifndef XM_ORT_GPU_EP
#define XM_ORT_GPU_EP "ROCMExecutionProvider"
#endif

namespace xm_ort {

constexpr const char *kDomain = "xmetai_plugins";   // reference register_op.cpp:20

// An OrtStatus becomes an exception carrying its message (reference
// ort_common.h ThrowIfFailed); ONNX Runtime reports exceptions thrown from a
// kernel's constructor or Compute as a failed status.
inline void ThrowIfFailed(const OrtApi &api, OrtStatus *st) {
    if (st != nullptr) {
        std::string msg = api.GetErrorMessage(st);
        api.ReleaseStatus(st);
        throw std::runtime_error(msg);
    }
}

inline void Check(int status, const char *err) {
    if (status != XM_OK) throw std::runtime_error(err);
}

// A missing attribute means the default (reference: attribute helpers, e.g.
// gated_deltanet2_fn_ort.cpp:163-185).
inline int64_t IntAttr(const OrtApi &api, const OrtKernelInfo *info, const char *name, int64_t dflt) {
    int64_t v = dflt;
    OrtStatus *st = api.KernelInfoGetAttribute_int64(info, name, &v);
    if (st != nullptr) {
        api.ReleaseStatus(st);
        v = dflt;
    }
    return v;
}

inline float FloatAttr(const OrtApi &api, const OrtKernelInfo *info, const char *name, float dflt) {
    float v = dflt;
    OrtStatus *st = api.KernelInfoGetAttribute_float(info, name, &v);
    if (st != nullptr) {
        api.ReleaseStatus(st);
        v = dflt;
    }
    return v;
}

// Borrowed view of an input (reference ort_common.h:74-101: shape, element
// type and data pointer; the element-type check happens in the C ABI).
inline xm_tensor_t Describe(const OrtApi &api, const OrtValue *value) {
    OrtTensorTypeAndShapeInfo *info = nullptr;
    ThrowIfFailed(api, api.GetTensorTypeAndShape(value, &info));
    size_t rank = 0;
    ONNXTensorElementDataType type = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
    OrtStatus *st = api.GetDimensionsCount(info, &rank);
    xm_tensor_t d{};
    if (st == nullptr && rank > XM_MAX_RANK) {
        api.ReleaseTensorTypeAndShapeInfo(info);
        throw std::runtime_error("tensor rank out of range");
    }
    if (st == nullptr) st = api.GetDimensions(info, d.shape, rank);
    if (st == nullptr) st = api.GetTensorElementType(info, &type);
    api.ReleaseTensorTypeAndShapeInfo(info);
    ThrowIfFailed(api, st);
    d.rank = static_cast<int32_t>(rank);
    // XM_ELEM_* take ONNX's values (FLOAT 1, INT64 7, FLOAT16 10, BFLOAT16 16)
    d.elem_type = static_cast<int32_t>(type);
    void *data = nullptr;
    ThrowIfFailed(api, api.GetTensorMutableData(const_cast<OrtValue *>(value), &data));
    d.data = data;
    return d;
}

// xm_allocator_t over ONNX Runtime's stream-aware scratch buffers (reference
// gated_deltanet2_fn_ort.cpp:89-111): alloc = KernelContext_GetScratchBuffer
// on the memory of input 0, free = the context allocator's Free.
struct ScratchAdapter {
    const OrtApi *api = nullptr;
    OrtKernelContext *ctx = nullptr;
    const OrtMemoryInfo *mem = nullptr;
    OrtAllocator *allocator = nullptr;

    static void *Alloc(void *self, size_t bytes) {
        auto *s = static_cast<ScratchAdapter *>(self);
        void *p = nullptr;
        OrtStatus *st = s->api->KernelContext_GetScratchBuffer(s->ctx, s->mem, bytes, &p);
        if (st != nullptr) {
            s->api->ReleaseStatus(st);
            return nullptr;
        }
        return p;
    }
    static void Free(void *self, void *p) {
        auto *s = static_cast<ScratchAdapter *>(self);
        if (p != nullptr) s->allocator->Free(s->allocator, p);
    }
};

// Optional outputs 1..count of an operator: the recurrent state after the
// last token.  count == 0 means the node's attributes do not ask for it.
constexpr int kMaxStateOutputs = 4;
struct StateOutputs {
    int count = 0;
    int32_t rank[kMaxStateOutputs] = {};
    int64_t shape[kMaxStateOutputs][XM_MAX_RANK] = {};
    const char *what = "";   // attribute that asks for it, for error messages
};

// Compute of a device operator: describe the inputs (between min_inputs and
// max_inputs of them; an omitted optional input reads as an empty tensor),
// validate (the C ABI writes the output shape and the scratch size), allocate
// output 0 (and the state outputs when the attributes ask for them), take the
// execution provider's compute stream, enqueue.  Nothing synchronises the
// host and nothing is cached on the kernel object.
//   state(in) -> StateOutputs
//   launch(in, n, &attrs, void *out, float *states[kMaxStateOutputs], stream, alloc, err, errlen) -> status
// (output 0 has the element type the op's descriptor declares for it)
template <typename Attrs, typename Validate, typename State, typename Launch>
void ComputeDeviceOp(const OrtApi &api, OrtKernelContext *ctx, size_t min_inputs, size_t max_inputs,
                     const Attrs &attrs, Validate validate, State state, Launch launch) {
    size_t n_inputs = 0;
    ThrowIfFailed(api, api.KernelContext_GetInputCount(ctx, &n_inputs));
    if (n_inputs < min_inputs || n_inputs > max_inputs) throw std::runtime_error("unexpected number of inputs");
    std::vector<xm_tensor_t> in(n_inputs);
    size_t n_bound = 0;   // inputs up to the last one the node binds
    for (size_t i = 0; i < n_inputs; ++i) {
        const OrtValue *v = nullptr;
        ThrowIfFailed(api, api.KernelContext_GetInput(ctx, i, &v));
        if (v == nullptr) {   // omitted optional input
            in[i] = xm_tensor_t{};
            in[i].rank = 1;
            in[i].elem_type = XM_ELEM_FLOAT;
            continue;
        }
        in[i] = Describe(api, v);
        n_bound = i + 1;
    }
    // Omitted optional inputs at the end (an empty input name in the graph)
    // read as absent, the same as a node with fewer inputs.
    n_inputs = std::max(n_bound, min_inputs);
    in.resize(n_inputs);
    char err[1024];
    int64_t out_shape[XM_MAX_RANK] = {};
    int32_t out_rank = 0;
    size_t scratch = 0;
    Check(validate(in.data(), n_inputs, &attrs, out_shape, &out_rank, &scratch, err, sizeof(err)), err);
    OrtValue *out = nullptr;
    ThrowIfFailed(api, api.KernelContext_GetOutput(ctx, 0, out_shape, static_cast<size_t>(out_rank), &out));
    void *out_data = nullptr;
    ThrowIfFailed(api, api.GetTensorMutableData(out, &out_data));

    size_t n_outputs = 0;
    ThrowIfFailed(api, api.KernelContext_GetOutputCount(ctx, &n_outputs));
    const StateOutputs so = state(in.data());
    float *states[kMaxStateOutputs] = {};
    if (so.count > 0) {
        if (n_outputs < static_cast<size_t>(1 + so.count))
            throw std::runtime_error(std::string(so.what) + "=1 needs " + std::to_string(so.count) +
                                     " state output(s) after output 0");
        for (int i = 0; i < so.count; ++i) {
            OrtValue *sv = nullptr;
            void *data = nullptr;
            ThrowIfFailed(api, api.KernelContext_GetOutput(ctx, 1 + i, so.shape[i], static_cast<size_t>(so.rank[i]), &sv));
            ThrowIfFailed(api, api.GetTensorMutableData(sv, &data));
            states[i] = static_cast<float *>(data);
        }
    } else if (n_outputs > 1) {
        throw std::runtime_error(std::string("outputs after output 0 (the state) need ") + so.what + "=1");
    }

    void *stream = nullptr;
    ThrowIfFailed(api, api.KernelContext_GetGPUComputeStream(ctx, &stream));

    ScratchAdapter s;
    s.api = &api;
    s.ctx = ctx;
    xm_allocator_t alloc{&s, &ScratchAdapter::Alloc, &ScratchAdapter::Free};
    const xm_allocator_t *ap = nullptr;
    if (scratch > 0) {
        const OrtValue *v0 = nullptr;
        ThrowIfFailed(api, api.KernelContext_GetInput(ctx, 0, &v0));
        ThrowIfFailed(api, api.GetTensorMemoryInfo(v0, &s.mem));
        ThrowIfFailed(api, api.KernelContext_GetAllocator(ctx, s.mem, &s.allocator));
        ap = &alloc;
    }
    const int st = launch(in.data(), n_inputs, &attrs, out_data, states, stream, ap, err,
                          sizeof(err));
    if (s.allocator != nullptr) api.ReleaseAllocator(s.allocator);
    Check(st, err);
}

}  // namespace xm_ort
