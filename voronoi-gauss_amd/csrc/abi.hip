// Error reporting of the C ABI (vgr_last_error) and the ABI version.
#include <cstdarg>
#include <cstdio>

#include "vgr_abi.h"

namespace vgr {

namespace {
thread_local char g_error[512] = "";
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

int launch_status(const char* kernel) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(VGR_ERR_LAUNCH, "%s: %s", kernel, hipGetErrorString(err));
    return VGR_OK;
}

}  // namespace vgr

extern "C" const char* vgr_last_error(void) { return vgr::g_error; }

extern "C" int vgr_abi_version(void) { return 27; }
