// Error state and version of the C ABI.
#include <cstdarg>

#include "common.h"

namespace moddit {
namespace {
thread_local char g_last_error[512] = {0};
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace moddit

extern "C" const char* moddit_last_error(void) { return moddit::g_last_error; }

extern "C" const char* moddit_version(void) { return "moddit-mi355x 0.1.0 (gfx950)"; }
