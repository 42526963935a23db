// Error reporting and library identity for the C ABI declared in include/leatmi.h.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace leat {

static thread_local char last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(last_error, sizeof(last_error), fmt, ap);
    va_end(ap);
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

}  // namespace leat

extern "C" const char* leat_last_error(void) { return leat::last_error; }

extern "C" int leat_abi_version(void) { return 2; }

// The compiled device architecture of this library's kernels, to check against the device.
extern "C" const char* leat_target(void) { return "gfx950"; }
