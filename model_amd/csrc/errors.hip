// Thread-local error reporting and version for the C ABI (include/mpl.h).
#include <stdarg.h>

#include "common.h"

namespace mpl {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace mpl

extern "C" int mpl_version(void) { return 100; }

extern "C" const char* mpl_last_error(void) { return mpl::g_err; }
