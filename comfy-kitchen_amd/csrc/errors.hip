// Thread-local error channel and version query of the C ABI.
#include <cstdarg>
#include <cstdio>

#include "ckh_common.h"

namespace ckh {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return CKH_ERR_LAUNCH;
    }
    return CKH_OK;
}

}  // namespace ckh

extern "C" int ckh_abi_version(void) { return CKH_ABI_VERSION; }

extern "C" const char* ckh_last_error(void) { return ckh::g_err; }
