// errors.cpp — the C ABI's per-thread last-error text (pocr_last_error) and
// fail(), through which every entry point returns its failure code.  Host
// code only, shared by the device runtime and the host-only sources.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/pocr_hip.h"

namespace pocr {

static thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

}  // namespace pocr

extern "C" const char *pocr_last_error(void) { return pocr::g_err.c_str(); }
