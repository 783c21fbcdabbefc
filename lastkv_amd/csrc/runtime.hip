// Error state and version of the C ABI.
#include "runtime.h"

#include <atomic>
#include <cstdio>

namespace lkv {

namespace {
thread_local char g_error[512] = "";
}

int32_t fail(int32_t status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int32_t check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(LKV_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
  return LKV_OK;
}

void clear_error() { g_error[0] = '\0'; }

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0 && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
    cached[dev].store(n, std::memory_order_relaxed);
  return n > 0 ? n : 0;
}

}  // namespace lkv

extern "C" int32_t lkv_abi_version(void) { return LKV_ABI_VERSION; }

extern "C" const char* lkv_last_error(void) { return lkv::g_error; }
