// Library-wide host helpers: the per-thread error message and the ABI version.
#include "sqx_common.h"

namespace sqx {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace sqx

extern "C" const char* sqx_last_error(void) { return sqx::g_last_error; }

extern "C" int sqx_abi_version(void) { return 2; }
