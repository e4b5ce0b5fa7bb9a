// C ABI support: per-thread error message and ABI version.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace abacus {
namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}
}  // namespace abacus

extern "C" {

const char* abacus_moe_last_error(void) { return abacus::g_error; }

int abacus_moe_abi_version(void) { return 5; }

}  // extern "C"
