// Quantized-KV decode attention (split over positions, log-sum-exp combine).
#include "common.h"

extern "C" size_t kvp_kv_decode_workspace_bytes(int, int, int, int, int) { return 0; }

extern "C" int kvp_kv_decode(const void*, const uint32_t*, const void*, const void*,
                             const uint32_t*, const void*, const void*, const void*, const void*,
                             const int32_t*, void*, int, int, int, int, int, int, int, int, int,
                             void*, size_t, void*) {
  return kvp::set_error(KVP_UNSUPPORTED, "kvp_kv_decode: not built yet");
}
