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

int device_cus()
{
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64 && cached[dev] > 0) return cached[dev];
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (dev < 64) cached[dev] = n;
    return n;
}

int pick_cpl(int64_t nch)
{
    static const int options[] = {1, 2, 3, 4, 6, 8, 10, 12, 16, 20, 24, 28, 32};
    for (int c : options)
        if ((int64_t)c * 64 >= nch) return c;
    return 0;
}

}  // namespace vdn

extern "C" const char* vdn_fp8_last_error(void) { return vdn::g_last_error; }

extern "C" int vdn_fp8_abi_version(void) { return VDN_FP8_ABI_VERSION; }
