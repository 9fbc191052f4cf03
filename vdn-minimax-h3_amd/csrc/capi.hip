// Host-side plumbing of the C ABI: the per-thread error message, launch
// checks and the ABI version.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

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

// The CU count of each device, queried once per device: only a successful query
// is kept (a failed one is retried by the next call), and concurrent first calls
// from several host threads at worst both query and store the same value.
namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];
}  // namespace

int device_cus()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < kMaxDevices) {
        const int cached = g_cus[dev].load(std::memory_order_relaxed);
        if (cached > 0) return cached;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    if (dev < kMaxDevices) g_cus[dev].store(n, std::memory_order_relaxed);
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

// The build's source manifest (JSON: sha256 of every source and header, of the
// flags, and their digest), injected by the build script.
#ifndef VDN_FP8_BUILD_INFO
#define VDN_FP8_BUILD_INFO "{}"
#endif
extern "C" const char* vdn_fp8_build_info(void) { return VDN_FP8_BUILD_INFO; }
