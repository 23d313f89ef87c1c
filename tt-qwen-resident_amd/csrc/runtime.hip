// Error reporting and version of libqwen_state.
#include <stdarg.h>
#include <stdio.h>

#include "qs_common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace qs {

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

// Status of the launch just enqueued: QS_EHIP with the HIP error text, or QS_OK.
int launch_status(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return QS_EHIP;
    }
    return QS_OK;
}

}  // namespace qs

extern "C" int qs_abi_version(void) { return 4; }

extern "C" const char *qs_last_error(void) { return g_err; }
