// Host-side runtime pieces shared by every entry point: thread-local error
// strings and the device-count helpers the planners use.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <string>

#include "common.h"

namespace mi355x {

namespace {
thread_local std::string g_last_error;
}

const char* set_error(const std::string& message) {
  g_last_error = message;
  return g_last_error.c_str();
}

const char* hip_error(hipError_t status, const char* what) {
  return set_error(std::string(what) + ": " + hipGetErrorString(status));
}

const char* launch_status(const char* what) {
  const hipError_t status = hipGetLastError();
  if (status == hipSuccess) return nullptr;
  return hip_error(status, what);
}

}  // namespace mi355x

extern "C" const char* mi355x_attn_error(void) { return mi355x::g_last_error.c_str(); }

extern "C" int mi355x_attn_abi_version(void) { return 1; }
