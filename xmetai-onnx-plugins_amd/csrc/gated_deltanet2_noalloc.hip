// GatedDeltaNet2Fn for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc):
// xm_gated_deltanet2_forward_noalloc.  It is xm_gated_deltanet2_forward with
// the scratch taken from a device array of fixed size instead of an
// allocator, and the same kernels.
//
// `scratch` below is a file-scope device array: each GPU the library runs on
// holds its own copy (64 MiB) from the library's first use on that device
// until the process ends.  In host code its name is only a stand-in for the
// symbol, so the address each device uses is looked up once per device with
// hipGetSymbolAddress and kept; kernels get that address.  The chunked
// windows and token chunks shrink to fit the array (GatedDeltaNet2ScratchBytes
// with a 64 MiB budget); a call that cannot fit even the smallest layout is
// rejected before anything is enqueued.  Nothing in the array has to start at
// zero: every region is written before it is read within one call.  Calls that
// overlap on one GPU share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "xm_common.h"
#include "xm_hip.h"
#include "xm_params.h"

namespace xm {
namespace {

constexpr size_t kNoAllocScratchBytes = size_t{64} << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];   // the array's address on each device, once looked up

// The array's address on the current device (looked up on the first call there).
void *ScratchOnCurrentDevice() {
    int dev = 0;
    XM_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) throw Error(XM_ERR_DEVICE, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *ptr = nullptr;
        XM_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (ptr == nullptr) throw Error(XM_ERR_DEVICE, "hipGetSymbolAddress returned a null address");
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace xm

extern "C" int xm_gated_deltanet2_forward_noalloc(const xm_tensor_t *inputs, size_t n_inputs,
                                                  const xm_gated_deltanet2_attrs_t *attrs, float *out, void *stream,
                                                  char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        xm::ResetLaunches();
        if (attrs == nullptr) xm::Invalid("attrs is null");
        if (attrs->output_final_state != 0)
            xm::Invalid("GatedDeltaNet2Fn with output_final_state=1 needs a final_state output "
                        "(xm_gated_deltanet2_forward_states)");
        const xm::GatedDeltaNet2Params p = xm::GatedDeltaNet2Plan(inputs, n_inputs, *attrs, out, nullptr);
        const size_t need = xm::GatedDeltaNet2ScratchBytes(p.batch, p.seqlen, p.nheads, p.dk, p.dv,
                                                           p.cu_seqlens != nullptr, xm::kNoAllocScratchBytes);
        if (need == SIZE_MAX)
            throw xm::Error(XM_ERR_UNSUPPORTED,
                            "GatedDeltaNet2Fn (xm_gated_deltanet2_forward_noalloc): the call needs more than the " +
                                std::to_string(xm::kNoAllocScratchBytes >> 20) +
                                " MiB of device scratch this entry point holds; use xm_gated_deltanet2_forward");
        void *buf = need > 0 ? xm::ScratchOnCurrentDevice() : nullptr;
        xm::LaunchGatedDeltaNet2(p, buf, need > 0 ? xm::kNoAllocScratchBytes : 0, stream);
    });
}
