// Thread-local error message behind hm_last_error(); no entry point aborts the process.
#include <cstdarg>

#include "common.h"

namespace hm {

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

}  // namespace hm

extern "C" const char* hm_last_error(void) { return hm::g_error; }
extern "C" int hm_abi_version(void) { return 1; }
