// Library identity and thread-local error reporting for the C ABI.
#include <string.h>

#include "abi_util.h"

namespace tbf16 {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace tbf16

extern "C" int tbf16_abi_version(void) { return TBF16_ABI_VERSION; }

extern "C" const char* tbf16_last_error(void) { return tbf16::g_err; }
