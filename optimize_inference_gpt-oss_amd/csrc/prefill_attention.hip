// placeholder
#include "gkv_device.hpp"
extern "C" int gkv_prefill_attention(void *, int32_t, const int32_t *, int32_t, int32_t, int32_t,
                                     const float *, int64_t, const void *, const void *,
                                     const float *, int32_t, void *, int64_t, int32_t) {
  return GKV_ERR_UNSUPPORTED;
}
