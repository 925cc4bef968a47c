// A stand-in for the parts of ONNX Runtime that a custom-op library meets:
// the OrtApi table (statuses, custom-op domains, kernel-info attributes, the
// kernel context's inputs, outputs, compute stream, scratch buffers and
// allocator, tensor type and shape), and a session's use of a registered
// operator (create the kernel from node attributes, run Compute on bound
// tensors, destroy the kernel).  Tensors are caller memory: the tests bind
// torch or NumPy buffers, outputs included, and read back the shapes the
// kernel asked for.  Exceptions that leave a kernel's constructor or Compute
// become the call's error, as ONNX Runtime reports them as failed statuses.
// Test infrastructure only; it is linked with the custom-op layer compiled
// against the headers beside it.
#include <cstdint>
#include <cstring>
#include <exception>
#include <map>
#include <string>
#include <vector>

#include "onnxruntime_c_api.h"

extern "C" OrtStatus *ORT_API_CALL RegisterCustomOps(OrtSessionOptions *options, const OrtApiBase *api_base);

struct OrtStatus {
    OrtErrorCode code;
    std::string msg;
};
struct OrtCustomOpDomain {
    std::string name;
    std::vector<const OrtCustomOp *> ops;
};
struct OrtSessionOptions {
    std::vector<OrtCustomOpDomain *> domains;
};
struct OrtKernelInfo {
    std::map<std::string, int64_t> ints;
    std::map<std::string, float> floats;
};
struct OrtMemoryInfo {
    bool device;
};
struct OrtValue {
    void *data = nullptr;
    std::vector<int64_t> shape;
    ONNXTensorElementDataType type = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
    bool device = false;
};
struct OrtTensorTypeAndShapeInfo {
    std::vector<int64_t> shape;
    ONNXTensorElementDataType type;
};

extern "C" {
// A tensor bound by the test: an input (present = 0 for an omitted optional
// input) or an output buffer of `capacity` bytes, whose shape the kernel's
// request is written back to.
typedef struct ortd_tensor {
    void *data;
    int64_t shape[8];
    int32_t rank;
    int32_t elem_type;
    int32_t present;
    int32_t device;
    uint64_t capacity;
} ortd_tensor_t;
}

struct OrtKernelContext {
    std::vector<OrtValue> inputs;
    std::vector<bool> present;
    ortd_tensor_t *outs = nullptr;
    int n_outs = 0;
    std::vector<OrtValue> out_values;
    const OrtCustomOp *op = nullptr;
    void *stream = nullptr;
    char *scratch = nullptr;
    size_t scratch_bytes = 0, scratch_used = 0, scratch_peak = 0;
    int frees = 0;
};

namespace {

const OrtMemoryInfo kDeviceMem{true}, kHostMem{false};

OrtStatus *Fail(OrtErrorCode code, const std::string &msg) { return new OrtStatus{code, msg}; }

size_t ElemBytes(ONNXTensorElementDataType t) {
    switch (t) {
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_DOUBLE:
            return 8;
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16:
            return 2;
        default:
            return 4;
    }
}

struct ContextAllocator : OrtAllocator {
    OrtKernelContext *ctx;
};

OrtApi MakeApi() {
    OrtApi a{};
    a.CreateStatus = [](OrtErrorCode code, const char *msg) { return Fail(code, msg ? msg : ""); };
    a.GetErrorCode = [](const OrtStatus *s) { return s ? s->code : ORT_OK; };
    a.GetErrorMessage = [](const OrtStatus *s) { return s ? s->msg.c_str() : ""; };
    a.ReleaseStatus = [](OrtStatus *s) { delete s; };
    a.CreateCustomOpDomain = [](const char *name, OrtCustomOpDomain **out) -> OrtStatus * {
        *out = new OrtCustomOpDomain{name ? name : "", {}};
        return nullptr;
    };
    a.CustomOpDomain_Add = [](OrtCustomOpDomain *d, const OrtCustomOp *op) -> OrtStatus * {
        if (op == nullptr || op->version > ORT_API_VERSION) return Fail(ORT_INVALID_ARGUMENT, "bad custom op");
        d->ops.push_back(op);
        return nullptr;
    };
    a.AddCustomOpDomain = [](OrtSessionOptions *o, OrtCustomOpDomain *d) -> OrtStatus * {
        o->domains.push_back(d);
        return nullptr;
    };
    a.KernelInfoGetAttribute_float = [](const OrtKernelInfo *info, const char *name, float *out) -> OrtStatus * {
        auto it = info->floats.find(name);
        if (it == info->floats.end()) return Fail(ORT_FAIL, std::string("No attribute with name:") + name);
        *out = it->second;
        return nullptr;
    };
    a.KernelInfoGetAttribute_int64 = [](const OrtKernelInfo *info, const char *name, int64_t *out) -> OrtStatus * {
        auto it = info->ints.find(name);
        if (it == info->ints.end()) return Fail(ORT_FAIL, std::string("No attribute with name:") + name);
        *out = it->second;
        return nullptr;
    };
    a.KernelContext_GetInputCount = [](const OrtKernelContext *c, size_t *out) -> OrtStatus * {
        *out = c->inputs.size();
        return nullptr;
    };
    a.KernelContext_GetOutputCount = [](const OrtKernelContext *c, size_t *out) -> OrtStatus * {
        *out = static_cast<size_t>(c->n_outs);
        return nullptr;
    };
    a.KernelContext_GetInput = [](const OrtKernelContext *c, size_t i, const OrtValue **out) -> OrtStatus * {
        if (i >= c->inputs.size()) return Fail(ORT_INVALID_ARGUMENT, "input index out of range");
        *out = c->present[i] ? &c->inputs[i] : nullptr;
        return nullptr;
    };
    a.KernelContext_GetOutput = [](OrtKernelContext *c, size_t i, const int64_t *dims, size_t n,
                                   OrtValue **out) -> OrtStatus * {
        if (i >= static_cast<size_t>(c->n_outs)) return Fail(ORT_INVALID_ARGUMENT, "output index out of range");
        if (n > 8) return Fail(ORT_INVALID_ARGUMENT, "output rank out of range");
        ortd_tensor_t &t = c->outs[i];
        const ONNXTensorElementDataType type = c->op->GetOutputType(c->op, i);
        size_t count = 1;
        for (size_t d = 0; d < n; ++d) {
            if (dims[d] < 0) return Fail(ORT_INVALID_ARGUMENT, "negative output dimension");
            count *= static_cast<size_t>(dims[d]);
            t.shape[d] = dims[d];
        }
        t.rank = static_cast<int32_t>(n);
        t.elem_type = type;
        t.present = 1;
        if (count * ElemBytes(type) > t.capacity) return Fail(ORT_FAIL, "output buffer too small");
        OrtValue &v = c->out_values[i];
        v.data = t.data;
        v.shape.assign(dims, dims + n);
        v.type = type;
        v.device = t.device != 0;
        *out = &v;
        return nullptr;
    };
    a.KernelContext_GetGPUComputeStream = [](const OrtKernelContext *c, void **out) -> OrtStatus * {
        *out = c->stream;
        return nullptr;
    };
    a.KernelContext_GetScratchBuffer = [](const OrtKernelContext *cc, const OrtMemoryInfo *mem, size_t bytes,
                                          void **out) -> OrtStatus * {
        auto *c = const_cast<OrtKernelContext *>(cc);
        *out = nullptr;
        if (mem == nullptr || !mem->device) return Fail(ORT_INVALID_ARGUMENT, "scratch requested off the device");
        const size_t at = (c->scratch_used + 255) / 256 * 256;
        if (bytes == 0) return nullptr;
        if (at + bytes > c->scratch_bytes) return Fail(ORT_FAIL, "scratch exhausted");
        *out = c->scratch + at;
        c->scratch_used = at + bytes;
        if (c->scratch_used > c->scratch_peak) c->scratch_peak = c->scratch_used;
        return nullptr;
    };
    a.KernelContext_GetAllocator = [](const OrtKernelContext *cc, const OrtMemoryInfo *, OrtAllocator **out) -> OrtStatus * {
        auto *al = new ContextAllocator{};
        al->version = ORT_API_VERSION;
        al->ctx = const_cast<OrtKernelContext *>(cc);
        al->Alloc = [](OrtAllocator *, size_t) -> void * { return nullptr; };
        al->Free = [](OrtAllocator *self, void *p) {
            if (p != nullptr) ++static_cast<ContextAllocator *>(self)->ctx->frees;
        };
        al->Info = [](const OrtAllocator *) { return &kDeviceMem; };
        *out = al;
        return nullptr;
    };
    a.ReleaseAllocator = [](OrtAllocator *al) { delete static_cast<ContextAllocator *>(al); };
    a.GetTensorTypeAndShape = [](const OrtValue *v, OrtTensorTypeAndShapeInfo **out) -> OrtStatus * {
        *out = new OrtTensorTypeAndShapeInfo{v->shape, v->type};
        return nullptr;
    };
    a.GetDimensionsCount = [](const OrtTensorTypeAndShapeInfo *i, size_t *out) -> OrtStatus * {
        *out = i->shape.size();
        return nullptr;
    };
    a.GetDimensions = [](const OrtTensorTypeAndShapeInfo *i, int64_t *dims, size_t n) -> OrtStatus * {
        for (size_t d = 0; d < n && d < i->shape.size(); ++d) dims[d] = i->shape[d];
        return nullptr;
    };
    a.GetTensorElementType = [](const OrtTensorTypeAndShapeInfo *i, ONNXTensorElementDataType *out) -> OrtStatus * {
        *out = i->type;
        return nullptr;
    };
    a.ReleaseTensorTypeAndShapeInfo = [](OrtTensorTypeAndShapeInfo *i) { delete i; };
    a.GetTensorMutableData = [](OrtValue *v, void **out) -> OrtStatus * {
        *out = v->data;
        return nullptr;
    };
    a.GetTensorMemoryInfo = [](const OrtValue *v, const OrtMemoryInfo **out) -> OrtStatus * {
        *out = v->device ? &kDeviceMem : &kHostMem;
        return nullptr;
    };
    return a;
}

const OrtApi g_api = MakeApi();
uint32_t g_requested_version = 0;
const OrtApiBase g_base = {[](uint32_t version) -> const OrtApi * {
                               g_requested_version = version;
                               return version <= ORT_API_VERSION ? &g_api : nullptr;
                           },
                           []() { return "xm-ort-double"; }};
// A runtime that is older than the headers: tables up to g_max_version only.
uint32_t g_max_version = ORT_API_VERSION;
const OrtApiBase g_old_base = {[](uint32_t version) -> const OrtApi * {
                                   return version <= g_max_version ? &g_api : nullptr;
                               },
                               []() { return "xm-ort-double-old"; }};
OrtSessionOptions g_options;
bool g_registered = false;

void Copy(char *err, size_t errlen, const std::string &msg) {
    if (err != nullptr && errlen > 0) {
        std::strncpy(err, msg.c_str(), errlen - 1);
        err[errlen - 1] = '\0';
    }
}

const OrtCustomOp *Op(int d, int i) {
    if (d < 0 || d >= static_cast<int>(g_options.domains.size())) return nullptr;
    const auto &ops = g_options.domains[d]->ops;
    return (i >= 0 && i < static_cast<int>(ops.size())) ? ops[i] : nullptr;
}

}  // namespace

extern "C" {

// Loads the library's operators as a session would (RegisterCustomOps with
// this runtime's OrtApiBase); once per process.  0 on success.
int ortd_register(char *err, size_t errlen) {
    if (g_registered) return 0;
    OrtStatus *st = RegisterCustomOps(&g_options, &g_base);
    if (st != nullptr) {
        Copy(err, errlen, st->msg);
        delete st;
        return 1;
    }
    g_registered = true;
    return 0;
}

// RegisterCustomOps with null session options or a null OrtApiBase: returns
// 1 if it reported an error status (message in err), 0 if it returned null.
int ortd_register_with_nulls(int null_options, int null_base, char *err, size_t errlen) {
    OrtSessionOptions scratch_options;
    OrtStatus *st = RegisterCustomOps(null_options ? nullptr : &scratch_options, null_base ? nullptr : &g_base);
    if (st == nullptr) return 0;
    Copy(err, errlen, st->msg);
    delete st;
    return 1;
}

// RegisterCustomOps against a runtime that gives API tables up to
// max_version only (0: none at all): returns 1 with the error status's
// message and code in err / *code, 0 if it returned null; *domains is the
// number of operator domains it added.
int ortd_register_with_max_version(uint32_t max_version, char *err, size_t errlen, int *code, int *domains) {
    OrtSessionOptions scratch_options;
    g_max_version = max_version;
    OrtStatus *st = RegisterCustomOps(&scratch_options, &g_old_base);
    g_max_version = ORT_API_VERSION;
    *domains = static_cast<int>(scratch_options.domains.size());
    if (st == nullptr) return 0;
    Copy(err, errlen, st->msg);
    *code = static_cast<int>(st->code);
    delete st;
    return 1;
}

uint32_t ortd_requested_api_version(void) { return g_requested_version; }
int ortd_domain_count(void) { return static_cast<int>(g_options.domains.size()); }
const char *ortd_domain_name(int d) {
    return (d >= 0 && d < ortd_domain_count()) ? g_options.domains[d]->name.c_str() : nullptr;
}
int ortd_op_count(int d) {
    return (d >= 0 && d < ortd_domain_count()) ? static_cast<int>(g_options.domains[d]->ops.size()) : -1;
}
uint32_t ortd_op_version(int d, int i) {
    const OrtCustomOp *op = Op(d, i);
    return op ? op->version : 0;
}
const char *ortd_op_name(int d, int i) {
    const OrtCustomOp *op = Op(d, i);
    return op ? op->GetName(op) : nullptr;
}
const char *ortd_op_ep(int d, int i) {
    const OrtCustomOp *op = Op(d, i);
    return op ? op->GetExecutionProviderType(op) : nullptr;
}
// Number of inputs (output = 0) or outputs (output = 1) of operator i.
int ortd_op_arity(int d, int i, int output) {
    const OrtCustomOp *op = Op(d, i);
    if (op == nullptr) return -1;
    return static_cast<int>(output ? op->GetOutputTypeCount(op) : op->GetInputTypeCount(op));
}
// Element type and characteristic of input/output `index`.
int ortd_op_slot(int d, int i, int output, int index, int *type, int *characteristic) {
    const OrtCustomOp *op = Op(d, i);
    if (op == nullptr) return -1;
    *type = output ? op->GetOutputType(op, index) : op->GetInputType(op, index);
    *characteristic = output ? op->GetOutputCharacteristic(op, index) : op->GetInputCharacteristic(op, index);
    return 0;
}

// One node of operator i of domain d: kernel created from the attributes
// (int and float), Compute over the bound inputs and output buffers on
// `stream` with `scratch` as the device scratch arena, kernel destroyed.
// Returns 0, 1 (the kernel constructor threw: an invalid node) or 2 (Compute
// threw: a failed Run); the message goes to err.  scratch_peak: the arena's
// high-water mark; frees: scratch buffers handed back through the allocator.
int ortd_run(int d, int i, int n_int, const char *const *int_names, const int64_t *int_vals, int n_float,
             const char *const *float_names, const float *float_vals, int n_in, const ortd_tensor_t *ins, int n_out,
             ortd_tensor_t *outs, void *stream, void *scratch, uint64_t scratch_bytes, uint64_t *scratch_peak,
             int *frees, char *err, size_t errlen) {
    const OrtCustomOp *op = Op(d, i);
    if (op == nullptr) {
        Copy(err, errlen, "no such operator");
        return 3;
    }
    OrtKernelInfo info;
    for (int k = 0; k < n_int; ++k) info.ints[int_names[k]] = int_vals[k];
    for (int k = 0; k < n_float; ++k) info.floats[float_names[k]] = float_vals[k];
    void *kernel = nullptr;
    try {
        kernel = op->CreateKernel(op, &g_api, &info);
    } catch (const std::exception &e) {
        Copy(err, errlen, e.what());
        return 1;
    }
    OrtKernelContext ctx;
    ctx.op = op;
    ctx.stream = stream;
    ctx.scratch = static_cast<char *>(scratch);
    ctx.scratch_bytes = scratch_bytes;
    ctx.outs = outs;
    ctx.n_outs = n_out;
    ctx.out_values.resize(static_cast<size_t>(n_out));
    for (int k = 0; k < n_out; ++k) outs[k].present = 0;
    ctx.inputs.resize(static_cast<size_t>(n_in));
    ctx.present.resize(static_cast<size_t>(n_in));
    for (int k = 0; k < n_in; ++k) {
        const ortd_tensor_t &t = ins[k];
        ctx.present[k] = t.present != 0;
        OrtValue &v = ctx.inputs[k];
        v.data = t.data;
        v.shape.assign(t.shape, t.shape + (t.rank < 0 ? 0 : t.rank > 8 ? 8 : t.rank));
        v.type = static_cast<ONNXTensorElementDataType>(t.elem_type);
        v.device = t.device != 0;
    }
    int rc = 0;
    try {
        op->KernelCompute(kernel, &ctx);
    } catch (const std::exception &e) {
        Copy(err, errlen, e.what());
        rc = 2;
    }
    op->KernelDestroy(kernel);
    if (scratch_peak != nullptr) *scratch_peak = ctx.scratch_peak;
    if (frees != nullptr) *frees = ctx.frees;
    return rc;
}

}  // extern "C"
