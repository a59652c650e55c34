// Library-level ABI: version, per-thread last error, expert geometry.
#include <hip/hip_runtime.h>

#include <string>

#include "pmoe_internal.h"

namespace pmoe {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

}  // namespace pmoe

extern "C" int pmoe_abi_version(void) { return PMOE_ABI_VERSION; }

extern "C" const char* pmoe_last_error(void) { return pmoe::g_last_error.c_str(); }

extern "C" int pmoe_geom_init(pmoe_geom* g, int hidden, int inter, int bits, int group) {
  pmoe::clear_error();
  if (!g) return pmoe::fail(PMOE_EINVAL, "geom_init: null pointer");
  if (bits != 4 && bits != 6) return pmoe::fail(PMOE_EINVAL, "geom_init: bits must be 4 or 6");
  if (group != 64) return pmoe::fail(PMOE_EINVAL, "geom_init: group must be 64");
  if (hidden <= 0 || inter <= 0 || hidden % 64 || inter % 64)
    return pmoe::fail(PMOE_EINVAL, "geom_init: hidden and inter must be positive multiples of 64");
  g->hidden = hidden;
  g->inter = inter;
  g->bits = bits;
  g->group = group;
  const int64_t up_w = int64_t(inter) * (int64_t(hidden) * bits / 32) * 4;
  const int64_t up_s = int64_t(inter) * (hidden / group) * 2;
  const int64_t dn_w = int64_t(hidden) * (int64_t(inter) * bits / 32) * 4;
  const int64_t dn_s = int64_t(hidden) * (inter / group) * 2;
  const int64_t sizes[PMOE_NCOMP] = {up_w, up_s, up_s, up_w, up_s, up_s, dn_w, dn_s, dn_s};
  int64_t off = 0;
  for (int c = 0; c < PMOE_NCOMP; ++c) {
    g->off[c] = off;
    g->nbytes[c] = sizes[c];
    off += (sizes[c] + 255) / 256 * 256;
  }
  g->expert_bytes = off;
  return PMOE_OK;
}
