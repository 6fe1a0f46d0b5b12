// Library-wide C-ABI helpers: error reporting and version.
#include <string.h>

#include "tx_host.h"

namespace tx {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace tx

extern "C" {

const char* tallax_last_error(void) { return tx::g_err; }

int tallax_abi_version(void) { return 1; }

}  // extern "C"
