// The ABI's bookkeeping: version and the calling thread's last error message.
#include <string>

#include "../../include/hsn_window.h"
#include "abi_util.h"

namespace hsn {
namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& message) { g_last_error = message; }
void clear_last_error() { g_last_error.clear(); }

}  // namespace hsn

extern "C" int hsn_win_abi_version(void) { return HSN_WINDOW_ABI_VERSION; }

extern "C" const char* hsn_win_last_error(void) { return hsn::g_last_error.c_str(); }
