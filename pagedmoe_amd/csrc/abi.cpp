// Library-level ABI: version, per-thread last error, expert geometry.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <vector>

#include "pmoe_internal.h"
#include "pmoe_kernels.h"

namespace pmoe {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

namespace {

struct Profiler {
  std::mutex mu;
  bool open = false;
  std::vector<hipEvent_t> events;   // 2 per record
  std::vector<int> ids;             // kernel id per record
  int used = 0;
  double total_ms[K_COUNT] = {};
  int64_t launches[K_COUNT] = {};
};

Profiler& prof() {
  static Profiler p;
  return p;
}

const char* kNames[K_COUNT] = {"router_logits", "route_select", "dispatch",  "qgemv_gateup",
                               "qgemv_down",    "combine",      "prefill_gateup", "prefill_down",
                               "decode_fused",  "decode_xcd",   "experts_xcd"};

}  // namespace

ProfScope::ProfScope(int id, hipStream_t st) : slot_(-1), st_(st) {
  Profiler& p = prof();
  if (!p.open) return;
  std::lock_guard<std::mutex> lk(p.mu);
  if (!p.open || p.used >= int(p.ids.size())) return;
  slot_ = p.used++;
  p.ids[slot_] = id;
  (void)hipEventRecord(p.events[2 * slot_], st_);
}

ProfScope::~ProfScope() {
  if (slot_ < 0) return;
  (void)hipEventRecord(prof().events[2 * slot_ + 1], st_);
}

}  // namespace pmoe

extern "C" int pmoe_profile_begin(int capacity) {
  pmoe::clear_error();
  pmoe::Profiler& p = pmoe::prof();
  std::lock_guard<std::mutex> lk(p.mu);
  if (p.open) return pmoe::fail(PMOE_ESTATE, "profile_begin: a profile is already open");
  if (capacity <= 0) return pmoe::fail(PMOE_EINVAL, "profile_begin: capacity must be positive");
  if (int(p.ids.size()) < capacity) {
    for (hipEvent_t e : p.events) (void)hipEventDestroy(e);
    p.events.assign(2 * size_t(capacity), nullptr);
    for (auto& e : p.events) PMOE_HIP(hipEventCreate(&e));
    p.ids.assign(capacity, 0);
  }
  p.used = 0;
  for (int i = 0; i < pmoe::K_COUNT; ++i) {
    p.total_ms[i] = 0.0;
    p.launches[i] = 0;
  }
  p.open = true;
  return PMOE_OK;
}

extern "C" int pmoe_profile_end(void) {
  pmoe::clear_error();
  pmoe::Profiler& p = pmoe::prof();
  std::lock_guard<std::mutex> lk(p.mu);
  if (!p.open) return pmoe::fail(PMOE_ESTATE, "profile_end: no open profile");
  p.open = false;
  for (int r = 0; r < p.used; ++r) {
    PMOE_HIP(hipEventSynchronize(p.events[2 * r + 1]));
    float ms = 0.0f;
    PMOE_HIP(hipEventElapsedTime(&ms, p.events[2 * r], p.events[2 * r + 1]));
    p.total_ms[p.ids[r]] += ms;
    p.launches[p.ids[r]] += 1;
  }
  return PMOE_OK;
}

extern "C" int pmoe_profile_kernels(void) { return pmoe::K_COUNT; }

extern "C" const char* pmoe_profile_name(int kernel) {
  return (kernel >= 0 && kernel < pmoe::K_COUNT) ? pmoe::kNames[kernel] : "";
}

extern "C" int pmoe_profile_read(int kernel, double* total_ms, int64_t* launches) {
  pmoe::clear_error();
  if (kernel < 0 || kernel >= pmoe::K_COUNT || !total_ms || !launches)
    return pmoe::fail(PMOE_EINVAL, "profile_read: bad argument");
  pmoe::Profiler& p = pmoe::prof();
  std::lock_guard<std::mutex> lk(p.mu);
  *total_ms = p.total_ms[kernel];
  *launches = p.launches[kernel];
  return PMOE_OK;
}

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
