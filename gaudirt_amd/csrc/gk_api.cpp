// Per-thread error state and version of the C ABI.
#include "gk_common.hpp"

namespace gk {
namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }
void clear_error() { g_last_error.clear(); }

}  // namespace gk

extern "C" const char* gk_last_error(void) { return gk::g_last_error.c_str(); }
extern "C" const char* gk_version(void) { return "gaudirt_amd 0.1.0 gfx950"; }
