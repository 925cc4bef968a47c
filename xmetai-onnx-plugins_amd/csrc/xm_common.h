// Host-side helpers shared by the three operators: tensor views, the
// error-to-status mapping of the C ABI, and the scratch allocator front end.
//
// The validation helpers mirror csrc/utils/ort_common.h:57-101 of the
// reference (row-major views, fp32 only, zero-element tensor = absent input).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <stdexcept>
#include <string>
#include <vector>

#include "xmetai_recurrent.h"

namespace xm {

// An error that maps to an xm_status_t at the C boundary.
class Error : public std::runtime_error {
public:
    Error(int status, const std::string &msg) : std::runtime_error(msg), status_(status) {}
    int status() const { return status_; }

private:
    int status_;
};

[[noreturn]] inline void Invalid(const std::string &msg) { throw Error(XM_ERR_INVALID_ARGUMENT, msg); }
[[noreturn]] inline void Unsupported(const std::string &msg) { throw Error(XM_ERR_UNSUPPORTED, msg); }

// Row-major fp32 view of one input (reference: TensorView, ort_common.h:57-62).
struct View {
    const float *data = nullptr;   // the address; 16-bit data where elem says so
    std::vector<int64_t> shape;
    size_t elements = 0;
    int32_t elem = XM_ELEM_FLOAT;
    bool present() const { return elements > 0; }
    size_t rank() const { return shape.size(); }
};

// allow_16bit: the SelectiveScanFn data tensors may also be float16 / bfloat16.
inline View MakeView(const xm_tensor_t &t, bool allow_16bit = false) {
    if (t.rank < 0 || t.rank > XM_MAX_RANK) Invalid("tensor rank out of range");
    const bool half = t.elem_type == XM_ELEM_FLOAT16 || t.elem_type == XM_ELEM_BFLOAT16;
    if (t.elem_type != XM_ELEM_FLOAT && !(allow_16bit && half))
        Invalid("TensorView expects float32 tensors");  // ort_common.h:90-92
    View v;
    v.elem = t.elem_type;
    v.shape.assign(t.shape, t.shape + t.rank);
    size_t n = 1;
    for (int64_t d : v.shape) {
        if (d < 0) Invalid("tensor dimension is negative");
        n *= static_cast<size_t>(d);
    }
    v.elements = n;
    if (n > 0) {
        if (t.data == nullptr) Invalid("non-empty tensor has a null data pointer");
        v.data = static_cast<const float *>(t.data);
    }
    return v;
}

// Borrowed int64 vector (cu_seqlens): rank 1, at least two entries.
struct IndexView {
    const int64_t *data = nullptr;
    int64_t count = 0;
};

inline IndexView MakeIndexView(const xm_tensor_t &t, const char *name) {
    if (t.elem_type != XM_ELEM_INT64) Invalid(std::string(name) + " must be an int64 tensor");
    if (t.rank != 1) Invalid(std::string(name) + " must have rank 1");
    if (t.shape[0] < 2) Invalid(std::string(name) + " must hold at least two offsets");
    if (t.data == nullptr) Invalid("non-empty tensor has a null data pointer");
    return IndexView{static_cast<const int64_t *>(t.data), t.shape[0]};
}

// Float views of the first `nfloat` inputs (all of them by default); the
// caller reads any others (cu_seqlens) with MakeIndexView.
inline std::vector<View> MakeViews(const xm_tensor_t *inputs, size_t n_inputs, size_t expected, const char *op,
                                   size_t nfloat = SIZE_MAX) {
    if (inputs == nullptr) Invalid(std::string(op) + " received a null input array");
    if (n_inputs != expected)
        Invalid(std::string(op) + " expects " + std::to_string(expected) + " inputs, got " + std::to_string(n_inputs));
    std::vector<View> v;
    const size_t nf = nfloat < expected ? nfloat : expected;
    v.reserve(nf);
    for (size_t i = 0; i < nf; ++i) v.push_back(MakeView(inputs[i]));
    return v;
}

inline void RequireRank(const View &v, size_t rank, const char *name) {
    if (v.rank() != rank) Invalid(std::string(name) + " must have rank " + std::to_string(rank));
}

inline void RequireSameShape(const View &a, const View &b, const char *an, const char *bn) {
    if (a.shape != b.shape) Invalid(std::string(an) + " shape must match " + bn);
}

// Positive dimension that fits int32 (reference: ToIntDim, gated_deltanet2_fn_ort.cpp:37-42).
inline int ToIntDim(int64_t value, const char *name) {
    if (value <= 0 || value > INT32_MAX) Invalid(std::string(name) + " dimension is out of range");
    return static_cast<int>(value);
}

inline void WriteShape(const std::vector<int64_t> &shape, int64_t *out_shape, int32_t *out_rank) {
    if (out_rank) *out_rank = static_cast<int32_t>(shape.size());
    if (out_shape)
        for (size_t i = 0; i < shape.size(); ++i) out_shape[i] = shape[i];
}

inline void WriteError(char *errbuf, size_t errlen, const char *msg) {
    if (errbuf == nullptr || errlen == 0) return;
    std::strncpy(errbuf, msg, errlen - 1);
    errbuf[errlen - 1] = '\0';
}

// Runs `fn`, converting exceptions into a status code and message.
template <typename Fn>
int Guard(char *errbuf, size_t errlen, Fn &&fn) {
    try {
        fn();
        WriteError(errbuf, errlen, "");
        return XM_OK;
    } catch (const Error &e) {
        WriteError(errbuf, errlen, e.what());
        return e.status();
    } catch (const std::exception &e) {
        WriteError(errbuf, errlen, e.what());
        return XM_ERR_DEVICE;
    } catch (...) {
        WriteError(errbuf, errlen, "unknown error");
        return XM_ERR_DEVICE;
    }
}

// Kernel-selection overrides, set through xm_set_kernel_override (tests and
// tuning); 0 everywhere means the dispatchers' own choice.  Read with one
// relaxed atomic load per launch.
enum Override {
    kOverrideGdn2Path,       // 1: GatedDeltaNet2Fn sequential fused kernel
    kOverrideGdn2Pairwise,   // 1: pairwise A and M in every chunk
    kOverrideGdn2Rows,       // rows of 16 lanes per value column of the fused kernel
    kOverrideM3Path,         // 1: Mamba3SisoFn token-by-token kernel
    kOverrideSsLpc,          // lanes per channel of the selective scan (dstate <= 16)
    kOverrideSsSplit,        // selective scan: 1 channel blocks only, 2 sequence-split
    kOverrideGdn2Kpw4,       // 1: GDN-2 chunked recurrence above 128 keys with 4 key tiles per wave, ceil(tiles/4) waves
    kOverrideGdn2Windowed,   // 1: GDN-2 chunked path in windows of 128 chunks (not sized to 128 MiB / one packed window)
    kOverrideGdn2Split,      // GDN-2 chunked path: 1 never split the sequence, 2 split it wherever it has 2+ chunks, 3 two unequal segments (the second two tiles per workgroup)
    kOverrideGdn2Ct,         // GDN-2 chunked recurrence: value-column tiles per workgroup (1 or 2)
    kOverrideCount
};
int64_t GetOverride(Override which);

// Per host thread, the kernels the current entry-point call has enqueued
// (reported by xm_last_launches): reset at the start of each forward call,
// which also clears a HIP error left on the thread by earlier calls.
void ResetLaunches();
void NoteLaunch(const char *name);
// "Base<a,b,...>" with the template arguments of one instantiation.
std::string KernelName(const char *base, std::initializer_list<const char *> types, std::initializer_list<int> args);
// Records one launch of an instantiation; the name is built once per call site
// and instantiation (a function-local static inside the launching template).
#define XM_NOTE_LAUNCH(base, types, ...)                                                    \
    do {                                                                                    \
        static const std::string xm_name_ = ::xm::KernelName(base, types, {__VA_ARGS__});   \
        ::xm::NoteLaunch(xm_name_.c_str());                                                 \
    } while (0)

// Stream-ordered scratch: forwards to the caller's allocator or to the
// library's default pool (defined in xm_runtime.hip).  Freed on scope exit;
// memory is reused only in stream order, so freeing right after the last
// launch is safe (reference: gated_deltanet2_fn_ort.cpp:89-111).
void *DefaultAlloc(size_t bytes, void *stream);
void *DefaultTryAlloc(size_t bytes, void *stream);   // nullptr when the pool cannot give the bytes
void DefaultFree(void *ptr, void *stream);

class Scratch {
public:
    Scratch(const xm_allocator_t *alloc, void *stream) : alloc_(alloc), stream_(stream) {}
    Scratch(const Scratch &) = delete;
    Scratch &operator=(const Scratch &) = delete;
    ~Scratch() {
        for (void *p : ptrs_) {
            if (alloc_ != nullptr) {
                if (alloc_->free) alloc_->free(alloc_->ctx, p);
            } else {
                DefaultFree(p, stream_);
            }
        }
    }
    void *Get(size_t bytes) {
        void *p = TryGet(bytes);
        if (p == nullptr && bytes > 0)
            throw Error(XM_ERR_ALLOC, "scratch allocation of " + std::to_string(bytes) + " bytes failed");
        return p;
    }
    // As Get, but nullptr when the allocator refuses the bytes (the caller
    // may then ask for a smaller layout).
    void *TryGet(size_t bytes) {
        if (bytes == 0) return nullptr;
        void *p = nullptr;
        if (alloc_ != nullptr) {
            if (alloc_->alloc == nullptr) throw Error(XM_ERR_ALLOC, "scratch allocator has no alloc callback");
            p = alloc_->alloc(alloc_->ctx, bytes);
        } else {
            p = DefaultTryAlloc(bytes, stream_);
        }
        if (p != nullptr) ptrs_.push_back(p);
        return p;
    }

private:
    const xm_allocator_t *alloc_;
    void *stream_;
    std::vector<void *> ptrs_;
};

}  // namespace xm
