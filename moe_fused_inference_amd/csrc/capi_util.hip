// capi_util.hip -- error reporting shared by every C-ABI entry point.
#include <stdarg.h>
#include <stdio.h>
#include "mx_host.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace mxh {
void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return (int)e;
    }
    return MXFP4_OK;
}
}  // namespace mxh

extern "C" int mxfp4_abi_version(void) { return MXFP4_HIP_ABI_VERSION; }
extern "C" const char* mxfp4_last_error(void) { return g_last_error; }
