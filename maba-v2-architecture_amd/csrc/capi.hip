// Error plumbing and small shared host helpers of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "maba_common.h"

#include <atomic>

namespace maba {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MABA_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return MABA_OK;
}

int device_cu_count() {
  static std::atomic<int> cache[64];   // zero-initialised (static storage); 0 = not queried yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

bool expect_shape(const maba_tensor* t, const char* name, int ndim, const int64_t* shape) {
  if (!t || !t->data) {
    set_error("%s: missing tensor", name);
    return false;
  }
  if (t->ndim != ndim) {
    set_error("%s: expected %dD tensor, got %dD", name, ndim, t->ndim);
    return false;
  }
  for (int i = 0; i < ndim; ++i) {
    if (shape[i] >= 0 && t->shape[i] != shape[i]) {
      set_error("%s: dim %d is %lld, expected %lld", name, i, (long long)t->shape[i], (long long)shape[i]);
      return false;
    }
  }
  return true;
}

bool expect_float(const maba_tensor* t, const char* name) {
  if (!is_float_dt(t->dtype)) {
    set_error("%s: unsupported dtype code %d (f32/f16/bf16 only)", name, t->dtype);
    return false;
  }
  return true;
}

}  // namespace maba

extern "C" const char* maba_hip_last_error(void) { return maba::g_last_error; }
extern "C" int maba_hip_abi_version(void) { return 1; }
