// Library-wide entry points: ABI version and the per-thread error message.
#include <cstring>

#include "tsa_common.h"

namespace tsa {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

const char* last_error() { return g_last_error; }

}  // namespace tsa

extern "C" int tsa_abi_version(void) { return TSA_ABI_VERSION; }

extern "C" const char* tsa_last_error(void) { return tsa::last_error(); }
