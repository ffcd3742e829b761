// status.hip -- error reporting shared by every libkvec entry point.
#include <cstdarg>
#include <cstdio>

#include "kvec_internal.h"

namespace kvec {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(KVEC_EHIP, "%s: %s", what, hipGetErrorString(e));
    return KVEC_OK;
}

}  // namespace kvec

extern "C" int kvec_version(void) { return 100; }

extern "C" const char* kvec_strerror(int code) {
    switch (code) {
        case KVEC_OK: return "success";
        case KVEC_EINVAL: return "invalid argument";
        case KVEC_EUNSUPPORTED: return "unsupported configuration";
        case KVEC_EHIP: return "HIP runtime error";
        case KVEC_EDECODE: return "erasure pattern cannot be decoded";
        default: return "unknown error";
    }
}

extern "C" const char* kvec_last_error(void) { return kvec::g_err; }

// Test hook for the invariant-divisor division used by the gather kernels
// (not part of the public header).
extern "C" uint32_t kvec_internal_fastdiv(uint32_t n, uint32_t d) {
    return kvec::fdiv(n, kvec::make_fastdiv(d));
}
