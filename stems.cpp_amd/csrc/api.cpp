// api.cpp — library-wide C entry points: version and the per-thread last-error message.
#include <string>

#include "common.hpp"

namespace stx {
namespace {
thread_local std::string g_last_error;
}
void set_last_error(const char* msg) { g_last_error = msg ? msg : ""; }
const char* last_error() { return g_last_error.c_str(); }
}  // namespace stx

extern "C" {
STX_API const char* stx_version(void) { return "0.2.0"; }
STX_API const char* stx_last_error(void) { return stx::last_error(); }
}
