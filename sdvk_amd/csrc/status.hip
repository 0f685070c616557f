// status.cpp -- status strings, thread-local error detail, version.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace mi {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return MI_OK;
}

}  // namespace mi

extern "C" const char* mi_status_string(int status) {
    switch (status) {
        case MI_OK: return "ok";
        case MI_ERR_INVALID_ARG: return "invalid argument";
        case MI_ERR_UNSUPPORTED: return "unsupported shape";
        case MI_ERR_ALIGNMENT: return "alignment requirement not met";
        case MI_ERR_ALIASING: return "output overlaps an input";
        case MI_ERR_HIP: return "HIP runtime error";
        case MI_ERR_IO: return "file or format error";
        case MI_ERR_NOT_FOUND: return "not found";
        default: return "unknown status";
    }
}

extern "C" const char* mi_last_error(void) { return g_last_error; }

extern "C" int mi_version(void) { return 100; /* 0.1.0 */ }
