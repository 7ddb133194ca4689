// ABI bookkeeping: version and the per-thread last-error string.
#include <stdarg.h>
#include <stdio.h>

#include "gdn_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

int gdn_set_error(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

void gdn_begin_call() { g_last_error[0] = '\0'; }

void gdn_begin_launches()
{
    // An error an earlier HIP call left pending on this thread (a previous framework op)
    // is drained, so that the checks after this call's launches report only their own,
    // and named in the last-error message, so that it is not lost: a call that then
    // succeeds returns GDN_OK with that note in gdn_last_error().
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        gdn_set_error(GDN_OK, "note: a HIP error left pending by an earlier call was cleared "
                      "before this call's launches: %s (%s)", hipGetErrorName(e),
                      hipGetErrorString(e));
}

int gdn_check_launch(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return gdn_set_error(GDN_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    return GDN_OK;
}

extern "C" int gdn_abi_version(void) { return GDN_HIP_ABI_VERSION; }

extern "C" const char *gdn_last_error(void) { return g_last_error; }
