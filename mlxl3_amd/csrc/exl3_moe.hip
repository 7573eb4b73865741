// MoE SwitchGLU entry points (grouped expert QMM); filled in with the kernels.
#include "../../include/exl3_hip.h"
#include "exl3_launch.hpp"

using namespace exl3;

struct exl3_moe {
  int dummy;
};

extern "C" {
int exl3_moe_create(const uint16_t*, const uint16_t*, const uint16_t*, const uint16_t*,
                    const uint16_t*, const uint16_t*, int32_t, int32_t, int32_t, int32_t, int32_t,
                    int32_t, exl3_moe** out_handle) {
  if (out_handle) *out_handle = nullptr;
  return fail(EXL3_EUNSUPPORTED, "MoE not built yet");
}
void exl3_moe_destroy(exl3_moe* h) { delete h; }
size_t exl3_moe_workspace_bytes(const exl3_moe*, int64_t) { return 0; }
int exl3_moe_forward(const exl3_moe*, const uint16_t*, int64_t, const uint32_t*, const uint16_t*,
                     uint16_t*, void*, size_t, void*) {
  return fail(EXL3_EUNSUPPORTED, "MoE not built yet");
}
}
