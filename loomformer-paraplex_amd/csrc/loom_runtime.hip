// Error plumbing and ABI version of libloom_hip.so.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <unordered_map>

#include "loom_common.h"

namespace loom {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// Report an asynchronous launch failure (bad grid, missing code object ...)
// that hipLaunchKernelGGL recorded for this thread.
int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
        return LOOM_ERR_LAUNCH;
    }
    return LOOM_OK;
}

// Compute units of the current device (cached per device).
int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
    return n;
}

// Threads of `kernel` (launched with `block` threads per block) that the
// current device holds resident at once: CUs x resident blocks per CU x block.
// Looked up once per (kernel, device) and cached.
int64_t resident_threads(const void* kernel, int block) {
    static std::mutex mu;
    static std::unordered_map<uint64_t, int64_t> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const uint64_t key = (uint64_t)(uintptr_t)kernel * 64u + (uint64_t)dev;
    {
        std::lock_guard<std::mutex> g(mu);
        auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    const int cus = device_cus();
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    const int64_t n = (int64_t)cus * per_cu * block;
    std::lock_guard<std::mutex> g(mu);
    cache[key] = n;
    return n;
}

}  // namespace loom

extern "C" const char* loom_last_error(void) { return loom::g_err; }

extern "C" int loom_abi_version(void) { return 10; }
