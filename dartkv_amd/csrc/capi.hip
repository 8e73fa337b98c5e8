// C ABI bookkeeping: version and the thread-local last-error string.
#include <stdarg.h>
#include <stdio.h>

#include "dkv_capi_util.h"

namespace dkv {
namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}
}  // namespace dkv

extern "C" const char* dkv_last_error(void) { return dkv::g_last_error; }

extern "C" int dkv_abi_version(void) { return 13; }
