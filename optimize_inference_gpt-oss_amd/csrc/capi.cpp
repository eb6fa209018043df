// Status strings and version of the gkv C ABI.
#include "gkv.h"

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
