// flare_capi.cpp -- error state and identification for the C ABI.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/flare_mi355x.h"

namespace flare {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return FLARE_ERR_LAUNCH;
    }
    return FLARE_OK;
}

}  // namespace flare

extern "C" {
int flare_abi_version(void) { return 1; }
const char* flare_last_error(void) { return flare::g_last_error; }
}
