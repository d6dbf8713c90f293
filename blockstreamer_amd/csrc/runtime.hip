// Error reporting and version of the C ABI.
#include <string.h>

#include "bsa_common.h"

namespace bsa {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace bsa

extern "C" const char* bsa_last_error(void) { return bsa::g_last_error; }

extern "C" int bsa_version(void) { return 302; }
