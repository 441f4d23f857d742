// Thread-local error message behind tfp8_last_error(), plus the ABI version query.
#include <stdarg.h>
#include <stdio.h>

#include "tfp8_common.h"

namespace tfp8 {

static thread_local char g_msg[512];

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_msg[0] = '\0'; }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
    return 0;
}

}  // namespace tfp8

extern "C" int tfp8_abi_version(void) { return TFP8_ABI_VERSION; }

extern "C" const char* tfp8_last_error(void) { return tfp8::g_msg; }
