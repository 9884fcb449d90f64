// Library-wide C-ABI entry points: version and thread-local error message.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <map>
#include <mutex>
#include <utility>

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
  static std::atomic<int> cached[64];   // zero-initialized (static storage)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

int pf_reserve_lds(const void* kernel, size_t bytes, const char* name) {
  // (kernel, device) -> status of the one hipFuncSetAttribute call made for it
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, hipError_t> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return pf_fail(PF_E_LAUNCH, "%s: cannot query the current device", name);
  hipError_t e;
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(kernel, dev);
    auto it = done.find(key);
    if (it == done.end())
      it = done.emplace(key, hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes)).first;
    e = it->second;
  }
  if (e != hipSuccess)
    return pf_fail(PF_E_LAUNCH, "%s: cannot reserve %zu bytes of LDS: %s", name, bytes, hipGetErrorString(e));
  return PF_OK;
}
