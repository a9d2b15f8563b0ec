// Host-side error state shared by every C-ABI entry point.
#include <string>

#include "fl_common.h"

namespace fl {
namespace {
thread_local std::string g_last_error;
}
void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }
}  // namespace fl

extern "C" const char* fl_last_error(void) { return fl::g_last_error.c_str(); }
extern "C" int32_t fl_abi_version(void) { return 4; }
