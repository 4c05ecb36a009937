// Error reporting and version entry points of the treeverify C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "tv_internal.h"

namespace tv {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
    va_end(args);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return fail(TV_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
    }
    return TV_OK;
}

}  // namespace tv

extern "C" int tv_abi_version(void) { return TV_ABI_VERSION; }

extern "C" const char* tv_last_error(void) { return tv::g_last_error; }

extern "C" int64_t tv_sizeof_tree_attention_args(void) {
    return static_cast<int64_t>(sizeof(tv_tree_attention_args));
}
