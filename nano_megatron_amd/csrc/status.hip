// Thread-local error reporting for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace nmb {

static thread_local char g_last_error[1024] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace nmb

extern "C" const char* nmb_last_error(void) { return nmb::g_last_error; }

extern "C" int nmb_abi_version(void) { return 2; }
