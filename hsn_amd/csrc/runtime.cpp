// The ABI's bookkeeping: version, the calling thread's last error message, and the per-kernel
// dynamic-LDS attribute record.
#include <hip/hip_runtime.h>

#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "../../include/hsn_window.h"
#include "abi_util.h"

namespace hsn {
namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& message) { g_last_error = message; }
void clear_last_error() { g_last_error.clear(); }

hipError_t allow_lds_raw(const void* kernel, size_t lds) {
    (void)lds;
    static std::mutex lock;
    static std::set<std::pair<const void*, int>> done;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> guard(lock);
    if (done.count({kernel, dev})) return hipSuccess;
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e == hipSuccess) done.insert({kernel, dev});
    return e;
}

}  // namespace hsn

extern "C" int hsn_win_abi_version(void) { return HSN_WINDOW_ABI_VERSION; }

extern "C" const char* hsn_win_last_error(void) { return hsn::g_last_error.c_str(); }
