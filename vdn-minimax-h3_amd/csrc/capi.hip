// Host-side plumbing of the C ABI: the per-thread error message, launch
// checks and the ABI version.
#include <stdarg.h>
#include <stdio.h>

#include "vdn_common.h"

namespace vdn {

static thread_local char g_last_error[512] = "";

int set_error(int status, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(VDN_FP8_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return VDN_FP8_OK;
}

}  // namespace vdn

extern "C" const char* vdn_fp8_last_error(void) { return vdn::g_last_error; }

extern "C" int vdn_fp8_abi_version(void) { return VDN_FP8_ABI_VERSION; }
