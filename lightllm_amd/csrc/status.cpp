// Thread-local error reporting for the C ABI; device occupancy queries.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <utility>

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

int device_cus() {
    static std::mutex mu;
    static std::map<int, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    cache[dev] = cus;
    return cus;
}

int resident_workgroups(const void* fn, int threads) {
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({dev, fn});
    if (it != cache.end()) return it->second;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const int cap = std::max(1, cus * per_cu);
    cache[{dev, fn}] = cap;
    return cap;
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

extern "C" int llkv_abi_version(void) { return 4; }
