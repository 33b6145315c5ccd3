// Status strings and per-thread error messages for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "gdn_common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace gdn_host {

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* kernel) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(GDN_ERR_HIP, "%s launch failed: %s", kernel, hipGetErrorString(err));
    g_last_error[0] = '\0';
    return GDN_OK;
}

}  // namespace gdn_host

extern "C" {

int gdn_abi_version(void) { return 1; }

const char* gdn_status_string(int status) {
    switch (status) {
        case GDN_OK: return "ok";
        case GDN_ERR_INVALID_ARGUMENT: return "invalid argument";
        case GDN_ERR_UNSUPPORTED: return "unsupported shape";
        case GDN_ERR_WORKSPACE: return "workspace too small";
        case GDN_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

const char* gdn_last_error(void) { return g_last_error; }

}  // extern "C"
