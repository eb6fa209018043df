// Status strings and version of the gkv C ABI.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <string>

#include "gkv.h"

namespace gkv {
static thread_local std::string g_last_error;

int hip_status(hipError_t e, const char *where) {
  if (e == hipSuccess)
    return GKV_OK;
  char buf[256];
  snprintf(buf, sizeof buf, "%s: %s (%d)", where, hipGetErrorString(e), (int)e);
  g_last_error = buf;
  return GKV_ERR_HIP;
}
} // namespace gkv

extern "C" const char *gkv_last_error(void) { return gkv::g_last_error.c_str(); }

extern "C" const char *gkv_status_string(int status) {
  switch (status) {
  case GKV_OK:
    return "ok";
  case GKV_ERR_ARG:
    return "bad argument";
  case GKV_ERR_UNSUPPORTED:
    return "unsupported shape";
  case GKV_ERR_CAPACITY:
    return "out of capacity";
  case GKV_ERR_BLOCK:
    return "invalid block or sequence id";
  case GKV_ERR_HIP:
    return "HIP runtime error";
  case GKV_ERR_WORKSPACE:
    return "workspace too small";
  default:
    return "unknown status";
  }
}

extern "C" const char *gkv_version(void) { return "0.1.0"; }
