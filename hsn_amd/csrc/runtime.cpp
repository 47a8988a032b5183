// The ABI's bookkeeping: version, the calling thread's last error message, and the per-kernel
// dynamic-LDS attribute record.
#include <hip/hip_runtime.h>

#include <mutex>
#include <map>
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
    static std::mutex lock;
    static std::map<std::pair<const void*, int>, size_t> room_of;  // dynamic LDS allowed
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> guard(lock);
    auto it = room_of.find({kernel, dev});
    if (it == room_of.end()) {
        // the CU's 160 KiB less the kernel's static LDS: a larger limit is refused
        hipFuncAttributes fa{};
        e = hipFuncGetAttributes(&fa, kernel);
        if (e != hipSuccess) return e;
        constexpr size_t kCuLds = 160 * 1024;
        if (fa.sharedSizeBytes > kCuLds) return hipErrorInvalidValue;
        const size_t room = kCuLds - fa.sharedSizeBytes;
        e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(room));
        if (e != hipSuccess) return e;
        it = room_of.emplace(std::make_pair(kernel, dev), room).first;
    }
    return lds <= it->second ? hipSuccess : hipErrorInvalidValue;
}

}  // namespace hsn

extern "C" int hsn_win_abi_version(void) { return HSN_WINDOW_ABI_VERSION; }

extern "C" const char* hsn_win_last_error(void) { return hsn::g_last_error.c_str(); }
