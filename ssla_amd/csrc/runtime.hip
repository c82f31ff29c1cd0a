// Library-wide runtime helpers: version and thread-local error messages.
#include "common.h"

#include <string.h>

namespace ssla {

static thread_local char g_last_error[512];

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace ssla

extern "C" int ssla_version(void) { return 100; }

extern "C" const char *ssla_last_error(void) { return ssla::g_last_error; }
