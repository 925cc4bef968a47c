// Library-wide runtime pieces: the default stream-ordered scratch pool and
// the version string.
#include <hip/hip_runtime.h>

#include <mutex>
#include <unordered_map>

#include "xm_common.h"
#include "xm_hip.h"

namespace xm {
namespace {

std::mutex g_pool_mu;
std::unordered_map<int, hipMemPool_t> g_pools;

// One pool per device, created on first use, never trimmed (release
// threshold = max), so steady-state calls do not map or unmap memory.
hipMemPool_t PoolForCurrentDevice() {
    int dev = 0;
    XM_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_pool_mu);
    auto it = g_pools.find(dev);
    if (it != g_pools.end()) return it->second;
    hipMemPoolProps props = {};
    props.allocType = hipMemAllocationTypePinned;
    props.handleTypes = hipMemHandleTypeNone;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t pool = nullptr;
    XM_HIP_CHECK(hipMemPoolCreate(&pool, &props));
    uint64_t threshold = ~0ull;
    XM_HIP_CHECK(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold));
    g_pools.emplace(dev, pool);
    return pool;
}

}  // namespace

void *DefaultAlloc(size_t bytes, void *stream) {
    hipMemPool_t pool = PoolForCurrentDevice();
    void *p = nullptr;
    XM_HIP_CHECK(hipMallocFromPoolAsync(&p, bytes, pool, static_cast<hipStream_t>(stream)));
    return p;
}

void DefaultFree(void *ptr, void *stream) {
    if (ptr != nullptr) (void)hipFreeAsync(ptr, static_cast<hipStream_t>(stream));
}

}  // namespace xm

extern "C" const char *xm_version(void) {
    return "xmetai-recurrent 0.1.0 (gfx950; SelectiveScanFn, Mamba3SisoFn, GatedDeltaNet2Fn)";
}
