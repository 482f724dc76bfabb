// Error state and version of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <map>
#include <mutex>
#include <utility>

#include "hif8_common.h"

namespace hif8 {

namespace {
thread_local char g_last_error[512] = {0};
}

int fail(int code, const char *fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char *what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(HIF8_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return HIF8_OK;
}

int reserve_dynamic_lds(const void *kernel, size_t bytes, const char *what) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess)
    return fail(HIF8_ERR_LAUNCH, "%s: no current HIP device", what);
  static std::mutex lock;
  static std::map<std::pair<const void *, int>, size_t> reserved;  // (kernel, device) -> bytes set
  std::lock_guard<std::mutex> guard(lock);
  size_t &have = reserved[std::make_pair(kernel, device)];
  if (bytes <= have) return HIF8_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)) != hipSuccess)
    return fail(HIF8_ERR_LAUNCH, "%s: cannot reserve %zu bytes of LDS", what, bytes);
  have = bytes;
  return HIF8_OK;
}

}  // namespace hif8

extern "C" const char *hif8_last_error(void) { return hif8::g_last_error; }

extern "C" int hif8_abi_version(void) { return 1; }
