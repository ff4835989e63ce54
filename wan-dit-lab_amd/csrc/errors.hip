// The error channel of the C ABI (a message per host thread, read with wdl_last_error()) and the device query the
// launchers share.
#include <stdarg.h>
#include <stdio.h>

#include "wdl_common.h"

namespace {
thread_local char g_message[1024] = "";
}

namespace wdl {

int fail(int code, const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_message, sizeof(g_message), fmt, args);
    va_end(args);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(WDL_EHIP, "%s: %s", what, hipGetErrorString(e));
    g_message[0] = 0;
    return WDL_OK;
}

int cu_count() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace wdl

extern "C" const char* wdl_last_error(void) { return g_message; }

extern "C" int wdl_abi_version(void) { return 14; }
