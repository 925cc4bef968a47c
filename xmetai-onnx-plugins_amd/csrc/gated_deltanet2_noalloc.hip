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
// zero: every region is written before it is read within one call.
//
// Calls on one GPU share the array.  Outside graph capture they are ordered:
// each waits on the device's event (hipStreamWaitEvent) before its kernels and
// records it after them, so a call on another stream starts only when the
// previous call's kernels are done (the event is created once per device,
// with the address lookup).  Under capture the call does neither, since a
// captured wait on an event recorded outside the capture is not allowed:
// replays of captured calls that overlap on one GPU, with each other or with
// eager calls, race on the array, and the caller orders them.
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

// The array's address on a device, looked up on the first call there, and
// the event that orders the calls using it.
struct DeviceScratch {
    void *ptr = nullptr;
    hipEvent_t last = nullptr;   // recorded after each uncaptured call's kernels
};
std::mutex g_scratch_mu;   // held from the lookup until a call's kernels and event record are enqueued
DeviceScratch g_scratch[kMaxDevices];

// The current device's array and event (set up on the first call there);
// g_scratch_mu must be held.
DeviceScratch &ScratchOnCurrentDevice() {
    int dev = 0;
    XM_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) throw Error(XM_ERR_DEVICE, "device ordinal out of range");
    DeviceScratch &d = g_scratch[dev];
    if (d.ptr == nullptr) {
        void *ptr = nullptr;
        XM_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (ptr == nullptr) throw Error(XM_ERR_DEVICE, "hipGetSymbolAddress returned a null address");
        hipEvent_t ev = nullptr;
        XM_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        d.ptr = ptr;
        d.last = ev;
    }
    return d;
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
        if (need == 0) {   // nothing touches the array
            xm::LaunchGatedDeltaNet2(p, nullptr, 0, stream);
            return;
        }
        std::lock_guard<std::mutex> lock(xm::g_scratch_mu);
        xm::DeviceScratch &d = xm::ScratchOnCurrentDevice();
        hipStream_t s = static_cast<hipStream_t>(stream);
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        XM_HIP_CHECK(hipStreamIsCapturing(s, &cs));
        const bool order = cs == hipStreamCaptureStatusNone;
        if (order) XM_HIP_CHECK(hipStreamWaitEvent(s, d.last, 0));
        xm::LaunchGatedDeltaNet2(p, d.ptr, xm::kNoAllocScratchBytes, stream);
        if (order) XM_HIP_CHECK(hipEventRecord(d.last, s));
    });
}
