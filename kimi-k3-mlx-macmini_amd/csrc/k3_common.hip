// Host-side error plumbing and small utility entry points.
#include <stdarg.h>
#include <stdio.h>

#include "k3_common.h"

namespace k3 {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int check_hip(hipError_t e, const char *what) {
    if (e == hipSuccess) return K3_OK;
    return set_error(K3_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace k3

extern "C" const char *k3_last_error(void) { return k3::g_err; }

extern "C" const char *k3_version(void) { return "k3hip 0.1 gfx950"; }
