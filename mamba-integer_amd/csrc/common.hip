// Status reporting and version of libmamba_int.
#include <stdarg.h>
#include <stdio.h>

#include "mi_common.hpp"

namespace mi {

static thread_local char g_error[512];

void clear_error() { g_error[0] = '\0'; }

mi_status fail(mi_status st, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return st;
}

mi_status check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return MI_OK;
}

}  // namespace mi

extern "C" const char *mi_version(void) { return "libmamba_int 0.2 (mi-spec-2, gfx950)"; }

extern "C" const char *mi_last_error_string(void) { return mi::g_error; }
