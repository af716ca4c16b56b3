// Error reporting and version entry points of libmeshy_amd.
#include <stdarg.h>
#include <stdio.h>

#include <hip/hip_runtime.h>

#include "common.h"

namespace meshy {

namespace {
thread_local char g_last_error[512] = {0};
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = 0; }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return set_error(static_cast<int>(e), "%s: %s", what, hipGetErrorString(e));
    }
    return MESHY_OK;
}

}  // namespace meshy

extern "C" const char* meshy_last_error(void) { return meshy::g_last_error; }

extern "C" int meshy_abi_version(void) { return 14; }

extern "C" int meshy_copy_to_device(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    meshy::clear_error();
    if (bytes == 0) return MESHY_OK;
    if (!dst || !src) return meshy::set_error(MESHY_ENULL, "meshy_copy_to_device: NULL pointer");
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess)
        return meshy::set_error(static_cast<int>(e), "meshy_copy_to_device: %s", hipGetErrorString(e));
    return MESHY_OK;
}
