// Host-side plumbing of the C ABI: the per-thread error message, launch
// checks and the ABI version.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

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

// The CU count of each device, queried once per device (std::call_once: calls
// from several host threads see one initialization and no torn value).
namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_cus_once[kMaxDevices];
int g_cus[kMaxDevices];
}  // namespace

int device_cus()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev >= kMaxDevices) {
        int n = 0;
        return hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? n : 0;
    }
    std::call_once(g_cus_once[dev], [dev]() {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
        g_cus[dev] = n;
    });
    return g_cus[dev];
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

// The build's source manifest (JSON: sha256 of every source and header, of the
// flags, and their digest), injected by the build script.
#ifndef VDN_FP8_BUILD_INFO
#define VDN_FP8_BUILD_INFO "{}"
#endif
extern "C" const char* vdn_fp8_build_info(void) { return VDN_FP8_BUILD_INFO; }
