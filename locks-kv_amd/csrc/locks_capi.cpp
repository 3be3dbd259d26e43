// C-ABI plumbing shared by every entry point: a thread-local error string
// and launch-status checking.  No entry point allocates device memory.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "locks_hip.h"

namespace locks {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -2;
    }
    return 0;
}

}  // namespace locks

extern "C" const char* locks_last_error(void) { return locks::g_err; }

extern "C" int32_t locks_abi_version(void) { return LOCKS_ABI_VERSION; }
