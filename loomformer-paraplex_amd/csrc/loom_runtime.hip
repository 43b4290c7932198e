// Error plumbing and ABI version of libloom_hip.so.
#include <cstdarg>
#include <cstdio>

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

}  // namespace loom

extern "C" const char* loom_last_error(void) { return loom::g_err; }

extern "C" int loom_abi_version(void) { return 1; }
