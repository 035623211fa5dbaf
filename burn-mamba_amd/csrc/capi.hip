// Library-wide C ABI helpers: error reporting and version.
#include "common.h"

namespace mamba {
static thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }
}  // namespace mamba

extern "C" const char* mamba_last_error(void) { return mamba::g_last_error.c_str(); }
extern "C" const char* mamba_version(void) { return "mamba_hip 0.2.0 gfx950"; }
