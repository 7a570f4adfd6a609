// Library-wide host state: thread-local error text and launch checks.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace {
thread_local char g_error[512] = "";
}

namespace reskv_host {

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error("%s failed: %s", what, hipGetErrorString(err));
        return 1;
    }
    return 0;
}

}  // namespace reskv_host

extern "C" const char* reskv_last_error(void) { return g_error; }

extern "C" int reskv_abi_version(void) { return 7; }
