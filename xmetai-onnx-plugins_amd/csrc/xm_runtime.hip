// Library-wide runtime pieces: the default stream-ordered scratch pool and
// the version string.
#include <hip/hip_runtime.h>

#include <algorithm>
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

namespace {
__global__ __launch_bounds__(256) void FillZerosKernel(float *dst, size_t count) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) dst[i] = 0.0f;
}
}  // namespace

void LaunchFillZeros(float *dst, size_t count, void *stream) {
    if (count == 0) return;
    const size_t blocks = std::min<size_t>((count + 255) / 256, 4096);
    hipLaunchKernelGGL(FillZerosKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dst, count);
    XM_LAUNCH_CHECK("zero fill");
}

}  // namespace xm

extern "C" const char *xm_version(void) {
    return "xmetai-recurrent 0.1.0 (gfx950; SelectiveScanFn, Mamba3SisoFn, GatedDeltaNet2Fn)";
}
