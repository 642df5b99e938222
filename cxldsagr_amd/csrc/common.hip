// C-ABI error channel and device queries shared by every entry point.
#include <stdarg.h>

#include "dsa_common.h"
#include "../../include/dsa_gfx950.h"

namespace dsa {

static thread_local char g_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
}

void clear_error() { g_error[0] = 0; }

int device_cu_count() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 256;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0)
    return 256;
  return cus;
}

}  // namespace dsa

extern "C" int dsa_last_error(char* buffer, size_t size) {
  if (buffer == nullptr || size == 0) return (int)strlen(dsa::g_error);
  snprintf(buffer, size, "%s", dsa::g_error);
  return (int)strlen(dsa::g_error);
}

extern "C" int dsa_abi_version(void) { return DSA_ABI_VERSION; }
