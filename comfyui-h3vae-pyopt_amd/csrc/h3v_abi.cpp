// Library-wide C-ABI plumbing: version, error strings.
#include "h3v_abi.hpp"

#include <stdarg.h>
#include <stdio.h>

namespace {
thread_local char g_last_error[1024] = "";
}

namespace h3v {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(H3V_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return H3V_OK;
}

}  // namespace h3v

extern "C" {

int h3v_abi_version(void) { return H3V_ABI_VERSION; }

const char* h3v_last_error(void) { return g_last_error; }

}  // extern "C"
