// Thread-local error reporting for the C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace llkv {

static thread_local char g_last_error[512] = "";

int set_error(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(LLKV_ERR_HIP, "%s: launch failed: %s", what,
                         hipGetErrorString(e));
    return LLKV_OK;
}

}  // namespace llkv

extern "C" const char* llkv_last_error(void) { return llkv::g_last_error; }

extern "C" const char* llkv_status_string(int status) {
    switch (status) {
        case LLKV_OK: return "ok";
        case LLKV_ERR_INVALID: return "invalid argument";
        case LLKV_ERR_UNSUPPORTED: return "unsupported configuration";
        case LLKV_ERR_WORKSPACE: return "workspace too small";
        case LLKV_ERR_HIP: return "HIP runtime error";
        case LLKV_ERR_EXHAUSTED: return "block pool exhausted";
    }
    return "unknown status";
}

extern "C" int llkv_abi_version(void) { return 2; }
