// Error state and device queries behind the C ABI (rk_last_error, rk_abi_version, rk_device_info).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <set>
#include <tuple>
#include <unordered_map>

#include "rk_internal.h"

namespace {
thread_local char g_err[1024] = "";
std::mutex g_cu_mutex;
std::unordered_map<int, int> g_cus;
std::mutex g_lds_mutex;
std::set<std::tuple<int, const void*, size_t>> g_lds_set;
}  // namespace

namespace rk {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(RK_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return RK_OK;
}

int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    auto it = g_cus.find(dev);
    if (it != g_cus.end()) return it->second;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    g_cus[dev] = n;
    return n;
}

int allow_dynamic_lds(const void* func, size_t bytes) {
    if (bytes <= 65536) return RK_OK;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(RK_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_lds_mutex);
    const auto key = std::make_tuple(dev, func, bytes);
    if (g_lds_set.count(key)) return RK_OK;
    e = hipFuncSetAttribute(func, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess)
        return fail(RK_ERR_HIP, "hipFuncSetAttribute(max dynamic LDS %zu): %s", bytes, hipGetErrorString(e));
    g_lds_set.insert(key);
    return RK_OK;
}

}  // namespace rk

extern "C" {

const char* rk_last_error(void) { return g_err; }

void rk_clear_error(void) { g_err[0] = '\0'; }

int rk_abi_version(void) { return RK_ABI_VERSION; }

int rk_device_info(int* compute_units, char* arch, int arch_len) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return rk::fail(RK_ERR_HIP, "no HIP device: %s", hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return rk::fail(RK_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (compute_units) *compute_units = prop.multiProcessorCount;
    if (arch && arch_len > 0) {
        strncpy(arch, prop.gcnArchName, (size_t)arch_len - 1);
        arch[arch_len - 1] = '\0';
    }
    return RK_OK;
}

}  // extern "C"
