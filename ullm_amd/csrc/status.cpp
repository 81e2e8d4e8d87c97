// Error string and version entry points of the C ABI.
#include <cstdarg>
#include <cstdio>
#include "../../include/ullm_hip.h"

namespace ullm {
static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace ullm

extern "C" const char *ullm_hip_version(void) { return "ullm-hip 0.1.0 gfx950"; }
extern "C" const char *ullm_hip_last_error(void) { return ullm::g_err; }
