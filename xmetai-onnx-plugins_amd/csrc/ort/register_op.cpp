// RegisterCustomOps: the symbol ONNX Runtime looks up when a session loads
// this library.  Reference: csrc/register_op.cpp:11-41 — domain
// "xmetai_plugins", operators added in the order SelectiveScanFn,
// Mamba3SisoFn, GatedDeltaNet2Fn, SoftmaxCPU, first failing status returned.
#include <string>

#include "ort_glue.h"
#include "xmetai_onnx_plugins_ort.h"

OrtStatus *XmAddSelectiveScanFnOp(const OrtApi &api, OrtCustomOpDomain *domain);
OrtStatus *XmAddMamba3SisoFnOp(const OrtApi &api, OrtCustomOpDomain *domain);
OrtStatus *XmAddGatedDeltaNet2FnOp(const OrtApi &api, OrtCustomOpDomain *domain);
OrtStatus *XmAddSoftmaxCpuOp(const OrtApi &api, OrtCustomOpDomain *domain);

namespace {

// The runtime is older than the headers this library was built with: no
// operator can be registered.  The newest table it does give (OrtApi only
// grows at its end, and CreateStatus is its first entry since version 1)
// carries the error back, so the session fails here, naming the versions,
// instead of later on an unknown operator.  Null when it gives no table.
OrtStatus *VersionMismatch(const OrtApiBase *api_base) {
    for (uint32_t v = ORT_API_VERSION - 1; v >= 1; --v) {
        const OrtApi *older = api_base->GetApi(v);
        if (older == nullptr) continue;
        const char *rt = api_base->GetVersionString != nullptr ? api_base->GetVersionString() : nullptr;
        const std::string msg = std::string(xm_ort::kDomain) + ": built for ONNX Runtime API version " +
                                std::to_string(ORT_API_VERSION) + ", but this runtime (" +
                                (rt != nullptr ? rt : "unknown version") + ") provides API version " +
                                std::to_string(v) + " at most";
        return older->CreateStatus(ORT_FAIL, msg.c_str());
    }
    return nullptr;
}

}  // namespace

extern "C" OrtStatus *ORT_API_CALL RegisterCustomOps(OrtSessionOptions *options, const OrtApiBase *api_base) {
    if (api_base == nullptr) return nullptr;
    const OrtApi *api = api_base->GetApi(ORT_API_VERSION);
    if (api == nullptr) return VersionMismatch(api_base);
    Ort::InitApi(api);                    // ORT_API_MANUAL_INIT: the C++ wrapper uses the runtime's table
    if (options == nullptr) return api->CreateStatus(ORT_INVALID_ARGUMENT, "RegisterCustomOps received null session options");
    OrtCustomOpDomain *domain = nullptr;
    OrtStatus *st = api->CreateCustomOpDomain(xm_ort::kDomain, &domain);
    if (st != nullptr) return st;
    using AddFn = OrtStatus *(*)(const OrtApi &, OrtCustomOpDomain *);
    const AddFn adds[] = {XmAddSelectiveScanFnOp, XmAddMamba3SisoFnOp, XmAddGatedDeltaNet2FnOp, XmAddSoftmaxCpuOp};
    for (AddFn add : adds) {
        st = add(*api, domain);
        if (st != nullptr) return st;
    }
    return api->AddCustomOpDomain(options, domain);
}
