// Host-side helpers of the C ABI: status codes, the thread's last error message, size checks.
//
// Every extern "C" entry point is wrapped in HSN_ABI_BEGIN / HSN_ABI_END so that no C++
// exception crosses the C boundary: a failed precondition returns its HSN_ERR_* code and
// records a message that hsn_win_last_error() returns.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>
#include <cstdio>
#include <initializer_list>
#include <string>

namespace hsn {

struct AbiError {
    int code;
    std::string message;
};

void set_last_error(const std::string& message);
void clear_last_error();

inline hipStream_t as_stream(void* stream) { return static_cast<hipStream_t>(stream); }

// The window entry points' bound on a whole tensor's element count: 64 * INT32_MAX (the kernels
// index across rows in int64 and within a row in int32). It is looser than the reference ABI's
// bound, every count <= INT32_MAX (kernels/include/hsn_ops.h:21-23), which the hsn_ops.h entry
// points (ops.hip, units.hip) check themselves.
inline bool check_elems(std::initializer_list<int64_t> counts) {
    for (int64_t c : counts)
        if (c < 0 || c > static_cast<int64_t>(INT32_MAX) * 64) return false;
    return true;
}

}  // namespace hsn

#define HSN_ABI_BEGIN \
    try {             \
        hsn::clear_last_error();

#define HSN_ABI_END                                                 \
    return HSN_OK;                                                  \
    }                                                               \
    catch (const hsn::AbiError& e) {                                \
        hsn::set_last_error(e.message);                             \
        return e.code;                                              \
    }                                                               \
    catch (...) {                                                   \
        hsn::set_last_error("unexpected C++ exception in the ABI"); \
        return HSN_ERR_BACKEND;                                     \
    }

#define HSN_REQUIRE(cond, code, msg)                          \
    do {                                                      \
        if (!(cond)) throw hsn::AbiError{(code), std::string(msg)}; \
    } while (0)

#define HSN_HIP(expr)                                                                    \
    do {                                                                                 \
        hipError_t err_ = (expr);                                                        \
        if (err_ != hipSuccess)                                                          \
            throw hsn::AbiError{HSN_ERR_BACKEND,                                         \
                                std::string(#expr) + ": " + hipGetErrorString(err_)};    \
    } while (0)
