// Library-wide C-ABI entry points: version and thread-local error message.
#include <stdarg.h>
#include <stdio.h>

#include "pf_internal.h"

namespace {
thread_local char g_last_error[512] = "";
}

int pf_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

extern "C" int pf_abi_version(void) { return PF_ABI_VERSION; }

extern "C" const char* pf_last_error(void) { return g_last_error; }

extern "C" int pf_operand_dtype(void) {
#ifdef PF_OPERAND_BF16
  return 1;
#else
  return 0;
#endif
}

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev] = cus;
  return cus;
}
