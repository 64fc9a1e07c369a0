// Library-level parts of the C ABI: status strings, per-thread error message,
// launch checking and the cached CU count.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "common.h"

namespace {
thread_local char g_last_error[512] = "";
std::mutex g_cu_mutex;
std::vector<int> g_cu_counts;
}  // namespace

namespace bc {

int set_error(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return BC_OK;
}

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    if ((int)g_cu_counts.size() <= dev) g_cu_counts.resize(dev + 1, 0);
    if (g_cu_counts[dev] == 0) {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cu <= 0)
            cu = 256;
        g_cu_counts[dev] = cu;
    }
    return g_cu_counts[dev];
}

}  // namespace bc

extern "C" int bc_abi_version(void) { return 1; }

extern "C" const char* bc_status_string(int status) {
    switch (status) {
        case BC_OK: return "ok";
        case BC_ERR_INVALID_ARGUMENT: return "invalid argument";
        case BC_ERR_UNSUPPORTED: return "unsupported";
        case BC_ERR_WORKSPACE: return "workspace too small";
        case BC_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

extern "C" const char* bc_last_error(void) { return g_last_error; }

// sizeof(BinaryVec) / sizeof(ResidualVec) of the reference (MAX_HEAD_DIM = 256):
// u32 words[8] + __half scale -> 34, padded to 36; u8 nibbles[128] + __half -> 130.
extern "C" int64_t bc_sizeof_binary_vec(void) { return 36; }
extern "C" int64_t bc_sizeof_residual_vec(void) { return 130; }
