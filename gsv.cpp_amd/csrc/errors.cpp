// Thread-local error message for the C ABI (gsvk_last_error).
#include <cstdarg>
#include <cstdio>

#include "gsvk.h"

namespace gsvk {

static thread_local char g_err[1024] = "";

void set_error(const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

const char * get_error() { return g_err; }

}  // namespace gsvk

extern "C" const char * gsvk_last_error(void) { return gsvk::get_error(); }
