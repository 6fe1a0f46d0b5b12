// Library-wide C-ABI helpers: error reporting and version.
#include <string.h>

#include <mutex>
#include <vector>

#include "tx_host.h"

namespace tx {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

hipError_t set_dynamic_lds_limit(const void* kernel, int bytes, hipStream_t stream) {
  struct Done {
    int dev;
    const void* kernel;
    int bytes;
  };
  static std::mutex mu;
  static std::vector<Done> done;
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  int dev = cur;
  if (stream && hipStreamGetDevice(stream, &dev) != hipSuccess) dev = cur;
  std::lock_guard<std::mutex> lock(mu);
  for (const Done& d : done)
    if (d.dev == dev && d.kernel == kernel && d.bytes >= bytes) return hipSuccess;
  if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return e;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (dev != cur) (void)hipSetDevice(cur);
  if (e == hipSuccess) done.push_back({dev, kernel, bytes});
  return e;
}

}  // namespace tx

extern "C" {

const char* tallax_last_error(void) { return tx::g_err; }

int tallax_abi_version(void) { return 2; }

}  // extern "C"
