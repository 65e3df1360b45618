// Thread-local last-error message of the C ABI.
#include "common.h"

namespace mep {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace mep

extern "C" const char* mep_last_error(void) { return mep::g_last_error; }

extern "C" int mep_abi_version(void) { return 2; }
