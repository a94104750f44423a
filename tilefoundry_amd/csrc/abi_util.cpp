// Status reporting for the C ABI: one thread-local message per calling thread.
#include "abi_util.h"

#include <string.h>

#include <mutex>

namespace {
thread_local char g_msg[512] = "";
}

namespace tfa {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

int launched(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TFA_ERR_LAUNCH, "%s: %s", kernel, hipGetErrorString(e));
  return TFA_OK;
}

int device_cus() {
  static std::mutex mu;
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int n = 0;
    cache[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cache[dev];
}

}  // namespace tfa

extern "C" {

const char* tfa_last_error(void) { return g_msg; }

const char* tfa_status_string(int status) {
  switch (status) {
    case TFA_OK: return "ok";
    case TFA_ERR_NULL: return "null pointer";
    case TFA_ERR_SHAPE: return "unsupported shape";
    case TFA_ERR_ALIGN: return "misaligned pointer";
    case TFA_ERR_CAPACITY: return "capacity exceeded";
    case TFA_ERR_ARG: return "invalid argument";
    case TFA_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

int tfa_abi_version(void) { return TFA_ABI_VERSION; }

}  // extern "C"
