// Library-wide runtime pieces: the default stream-ordered scratch pool, the
// once-per-device kernel attributes, the kernel-selection overrides and the
// version string.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>

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

void *DefaultTryAlloc(size_t bytes, void *stream) {
    hipMemPool_t pool = PoolForCurrentDevice();
    void *p = nullptr;
    if (hipMallocFromPoolAsync(&p, bytes, pool, static_cast<hipStream_t>(stream)) != hipSuccess) {
        (void)hipGetLastError();   // this call's own error
        return nullptr;
    }
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
    XM_NOTE_LAUNCH("FillZerosKernel", {}, );
    hipLaunchKernelGGL(FillZerosKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dst, count);
    XM_LAUNCH_CHECK("zero fill");
}

namespace {
// Packed sequences: zeros the token rows of `out` ([seqlen][row_floats]) that
// no sequence covers.  Sequence b covers [lo_b, hi_b), lo_b = clamp(cu[b]),
// hi_b = clamp(max(cu[b + 1], lo_b)), the ranges the operator kernels use;
// non-decreasing offsets cover exactly [lo_0, hi_{n-1}), other offsets are
// checked sequence by sequence (malformed input: time linear in n per row).
// A workgroup takes rows blockIdx.x, blockIdx.x + gridDim.x, ...
__global__ __launch_bounds__(256) void PackedGapsKernel(float *out, size_t row_floats, const int64_t *cu, int n,
                                                        int seqlen) {
    __shared__ int s_monotone;
    if (threadIdx.x == 0) s_monotone = 1;
    __syncthreads();
    bool mono = true;
    for (int b = threadIdx.x; b < n; b += blockDim.x) mono = mono && cu[b] <= cu[b + 1];
    if (!mono) s_monotone = 0;
    __syncthreads();
    const bool monotone = s_monotone != 0;
    const long long L = seqlen;
    auto clampt = [&](long long x) { return min(max(x, 0LL), L); };
    const long long first = clampt(cu[0]), last = clampt(max(cu[n], first));
    for (long long t = blockIdx.x; t < L; t += gridDim.x) {   // workgroup-uniform
        bool covered = false;
        if (monotone) {
            covered = t >= first && t < last;
        } else {
            for (int b = 0; b < n && !covered; ++b) {
                const long long lo = clampt(cu[b]), hi = clampt(max(cu[b + 1], lo));
                covered = t >= lo && t < hi;
            }
        }
        if (!covered)
            for (size_t i = threadIdx.x; i < row_floats; i += blockDim.x) out[static_cast<size_t>(t) * row_floats + i] = 0.0f;
    }
}
}  // namespace

void LaunchPackedGaps(float *out, size_t row_floats, const int64_t *cu, int n, int seqlen, void *stream) {
    if (seqlen <= 0 || row_floats == 0) return;
    const int blocks = std::min(seqlen, 1024);
    XM_NOTE_LAUNCH("PackedGapsKernel", {}, );
    hipLaunchKernelGGL(PackedGapsKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), out, row_floats, cu, n, seqlen);
    XM_LAUNCH_CHECK("packed sequence gaps");
}

namespace {
std::mutex g_attr_mu;
std::map<std::pair<const void *, int>, int> g_dyn_lds;   // (kernel, device) -> dynamic LDS limit set
}  // namespace

void EnsureDynamicLds(const void *kernel, int bytes) {
    int dev = 0;
    XM_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_attr_mu);
    int &set = g_dyn_lds[{kernel, dev}];
    if (bytes <= set) return;
    XM_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    set = bytes;
}

namespace {
struct OverrideSpec {
    const char *name;
    int64_t allowed[6];   // accepted non-default values, 0-terminated
};
// Index order of the Override enum.
constexpr OverrideSpec kOverrides[kOverrideCount] = {
    {"gdn2_path", {1, 0}},               // 1: the sequential fused kernel
    {"gdn2_pairwise", {1, 0}},           // 1: pairwise A and M in every chunk
    {"gdn2_rows", {1, 2, 4, 0}},         // rows of 16 lanes per value column (sequential kernel)
    {"m3_path", {1, 0}},                 // 1: the token-by-token kernel
    {"ss_lpc", {1, 2, 4, 8, 16, 0}},     // lanes per channel (dstate <= 16)
    {"ss_split", {1, 2, 0}},             // 1: one workgroup per channel block; 2: sequence-split
    {"gdn2_kpw4", {1, 0}},               // 1: GDN-2 chunked, 4 key tiles per wave above 128 keys
    {"gdn2_windowed", {1, 0}},           // 1: GDN-2 chunked, windows of 128 chunks only
    {"gdn2_split", {1, 2, 3, 0}},        // GDN-2 chunked: 1 no sequence split, 2 split wherever 2+ chunks,
                                         // 3 two unequal segments, the second at two tiles per workgroup
    {"gdn2_ct", {1, 2, 0}},              // GDN-2 chunked: 1 or 2 value-column tiles per recurrence workgroup
};
std::atomic<int64_t> g_override[kOverrideCount];

int FindOverride(const char *name) {
    if (name == nullptr) return -1;
    for (int i = 0; i < kOverrideCount; ++i)
        if (std::strcmp(name, kOverrides[i].name) == 0) return i;
    return -1;
}
}  // namespace

int64_t GetOverride(Override which) { return g_override[which].load(std::memory_order_relaxed); }

namespace {
struct LaunchLog {
    const char *names[16];
    int counts[16];
    int n = 0;
    std::string text;
};
thread_local LaunchLog t_launches;
thread_local hipError_t t_entry_error = hipSuccess;   // pending when the current call began
}  // namespace

void ResetLaunches() {
    t_launches.n = 0;
    // hipGetLastError reports the last error of any runtime call on this
    // thread, including the caller's own (a framework probing devices leaves
    // one behind), and clears it.  Note it without clearing: the launch
    // checks of this call take only an error that differs from it, and the
    // caller still finds its own.
    t_entry_error = hipPeekAtLastError();
}

hipError_t TakeLaunchError() {
    const hipError_t e = hipPeekAtLastError();
    if (e == hipSuccess || e == t_entry_error) return hipSuccess;
    return hipGetLastError();
}

void NoteLaunch(const char *name) {
    LaunchLog &l = t_launches;
    for (int i = 0; i < l.n; ++i)
        if (l.names[i] == name) {
            ++l.counts[i];
            return;
        }
    if (l.n < 16) {
        l.names[l.n] = name;
        l.counts[l.n++] = 1;
    }
}

std::string KernelName(const char *base, std::initializer_list<const char *> types, std::initializer_list<int> args) {
    std::string s = base;
    if (types.size() + args.size() == 0) return s;
    s += '<';
    bool first = true;
    for (const char *t : types) {
        s += first ? "" : ",";
        s += t;
        first = false;
    }
    for (int a : args) {
        s += first ? "" : ",";
        s += std::to_string(a);
        first = false;
    }
    return s + '>';
}

}  // namespace xm

extern "C" int xm_set_kernel_override(const char *name, int64_t value, char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        const int i = xm::FindOverride(name);
        if (i < 0) xm::Invalid(std::string("unknown kernel override ") + (name ? name : "(null)"));
        bool ok = value == 0;
        for (int64_t v : xm::kOverrides[i].allowed) ok = ok || (v != 0 && v == value);
        if (!ok) xm::Invalid(std::string("value out of range for kernel override ") + name);
        xm::g_override[i].store(value, std::memory_order_relaxed);
    });
}

extern "C" int64_t xm_get_kernel_override(const char *name) {
    const int i = xm::FindOverride(name);
    return i < 0 ? -1 : xm::g_override[i].load(std::memory_order_relaxed);
}

extern "C" const char *xm_last_launches(void) {
    xm::LaunchLog &l = xm::t_launches;
    l.text.clear();
    for (int i = 0; i < l.n; ++i) {
        if (i) l.text += ';';
        l.text += l.names[i];
        if (l.counts[i] > 1) l.text += " x" + std::to_string(l.counts[i]);
    }
    return l.text.c_str();
}

extern "C" const char *xm_version(void) {
    return "xmetai-recurrent 0.1.0 (gfx950; SelectiveScanFn, Mamba3SisoFn, GatedDeltaNet2Fn)";
}
