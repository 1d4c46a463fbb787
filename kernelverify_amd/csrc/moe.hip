// MoE routing, token permutation, gather-qmv dispatch.
#include "common.h"

extern "C" int kvp_moe_route(const void*, const void*, uint32_t*, float*, int, int, int, int,
                             void*) {
  return kvp::set_error(KVP_UNSUPPORTED, "kvp_moe_route: not built yet");
}
extern "C" int kvp_moe_route_logits(const float*, uint32_t*, float*, int, int, int, void*) {
  return kvp::set_error(KVP_UNSUPPORTED, "kvp_moe_route_logits: not built yet");
}
extern "C" int kvp_moe_permute(const uint32_t*, int32_t*, int32_t*, int, int, int, void*) {
  return kvp::set_error(KVP_UNSUPPORTED, "kvp_moe_permute: not built yet");
}
extern "C" int kvp_moe_dispatch(const void*, const uint32_t*, const float*, const uint32_t*,
                                const void*, const void*, void*, int, int, int, int, int, int, int,
                                void*) {
  return kvp::set_error(KVP_UNSUPPORTED, "kvp_moe_dispatch: not built yet");
}
extern "C" size_t kvp_moe_swiglu_workspace_bytes(int, int, int, int, int) { return 0; }
extern "C" int kvp_moe_swiglu(const void*, const uint32_t*, const float*, const uint32_t*,
                              const void*, const void*, const uint32_t*, const void*, const void*,
                              const uint32_t*, const void*, const void*, void*, int, int, int, int,
                              int, int, int, void*, size_t, void*) {
  return kvp::set_error(KVP_UNSUPPORTED, "kvp_moe_swiglu: not built yet");
}
