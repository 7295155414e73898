// errors.cpp — the calling thread's last failure message and the library
// version (host code of libnavi_trace.so; the host-only sanitizer build links
// it with relayout.cpp).
#include <cstdarg>
#include <cstdio>

#include "navi_trace.h"

namespace navi {

thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

}  // namespace navi

extern "C" const char* navi_last_error(void) { return navi::g_last_error; }

extern "C" const char* navi_version(void) { return "0.3.0"; }
