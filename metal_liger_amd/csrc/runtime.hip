// Library-wide state: ABI version, thread-local error string, device queries.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "common.h"

namespace mla {

namespace {
thread_local char g_last_error[1024] = "";
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices] = {0};
std::once_flag g_cus_once[kMaxDevices];
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(g_cus_once[dev], [dev]() {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cus[dev] = n;
  });
  return g_cus[dev];
}

}  // namespace mla

extern "C" int ml_abi_version(void) { return ML_ABI_VERSION; }

extern "C" const char* ml_last_error(void) { return mla::g_last_error; }
