// Version and error reporting of the C ABI (include/sparse_attn.h).
#include <stdarg.h>
#include <stdio.h>

#include "sa_common.h"

namespace sa {

static thread_local char g_last_error[512] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

}  // namespace sa

extern "C" int sa_abi_version(void) { return SA_ABI_VERSION; }

extern "C" const char* sa_last_error(void) { return sa::g_last_error; }
