// Error reporting for the C ABI: status codes plus a thread-local message.
#pragma once
#include <hip/hip_runtime.h>
#include <stdio.h>

#include "../../include/dartkv.h"

namespace dkv {
// Defined in capi.hip.
void set_error(const char* fmt, ...);
}  // namespace dkv

#define DKV_CHECK(cond, code, ...)   \
  do {                               \
    if (!(cond)) {                   \
      dkv::set_error(__VA_ARGS__);   \
      return (code);                 \
    }                                \
  } while (0)

// Report a failed kernel launch (bad configuration, no device, ...).
static inline int dkv_check_launch(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    dkv::set_error("%s: kernel launch failed: %s", where, hipGetErrorString(e));
    return DKV_ERR_HIP;
  }
  return DKV_OK;
}
