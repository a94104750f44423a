// Host-side helpers shared by the extern "C" entry points: argument checks that
// turn into status codes, and the thread-local message tfa_last_error() reports.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tilefoundry_amd.h"

namespace tfa {

// Records a message for tfa_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);

// Checks the launch that was just issued; on failure records
// "<kernel>: <hip error string>" and returns TFA_ERR_LAUNCH.
int launched(const char* kernel);

// Compute units of the current device, read once per device (256 if the query fails).
int device_cus();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

}  // namespace tfa

#define TFA_REQUIRE(cond, code, ...) \
  do {                               \
    if (!(cond)) return ::tfa::fail((code), __VA_ARGS__); \
  } while (0)

#define TFA_NONNULL(p) TFA_REQUIRE((p) != nullptr, TFA_ERR_NULL, "%s: null pointer '%s'", __func__, #p)
#define TFA_ALIGN16(p) TFA_REQUIRE(::tfa::aligned16(p), TFA_ERR_ALIGN, "%s: '%s' is not 16-byte aligned", __func__, #p)
