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

static void span_label(const Span& s, char* buf, size_t n) {
    if (s.idx >= 0) snprintf(buf, n, "%s[%d]", s.name, s.idx);
    else snprintf(buf, n, "%s", s.name);
}

int check_no_alias(const Span* w, int nw, const Span* r, int nr, const char* fn) {
    for (int i = 0; i < nw; ++i) {
        const Span* hit = nullptr;
        for (int j = i + 1; j < nw && !hit; ++j)
            if (ranges_overlap(w[i].p, w[i].n, w[j].p, w[j].n)) hit = &w[j];
        for (int j = 0; j < nr && !hit; ++j)
            if (ranges_overlap(w[i].p, w[i].n, r[j].p, r[j].n)) hit = &r[j];
        if (hit) {
            char a[64], b[64];
            span_label(w[i], a, sizeof a);
            span_label(*hit, b, sizeof b);
            return set_error(KVEC_EINVAL, "%s: %s overlaps %s", fn, a, b);
        }
    }
    return KVEC_OK;
}

}  // namespace kvec

extern "C" int kvec_version(void) { return KVEC_VERSION; }

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
