// Prefill expert GEMM (placeholder until the MFMA path lands).
#include "pmoe_internal.h"
#include "pmoe_kernels.h"

namespace pmoe {

int prefill_tile_m() { return 128; }

bool prefill_wanted(const pmoe_geom*, int, int, int) { return false; }

int prefill_experts(const pmoe_geom*, const uint8_t*, const int32_t*, int, int, const uint16_t*,
                    int, int, const int32_t*, const int32_t*, const int32_t*, const int2*,
                    const int32_t*, int, uint16_t*, void*, int, hipStream_t) {
  return fail(PMOE_EINVAL, "prefill path not built");
}

}  // namespace pmoe
