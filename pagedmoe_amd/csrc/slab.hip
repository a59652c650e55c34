// Expert slab slot table: residency policy on the host, table on the device.
//
// Restates ExpertCache's slab policy (cache.py:410): free list popped LIFO so
// the first allocation is slot 0 (:991, :1138-1139); a reserve of
// max(4, int(slots*reserve_frac)) slots kept out of the resident budget
// (:996-1002); per decode layer step: clear pins, classify ids (hit -> MRU,
// freq = min(8, freq+1), pin), give each miss a free slot or evict the least
// recent unpinned non-stitch entry (_alloc_slot :1118-1159), install misses
// with the LFRU second-chance trim (_install :2293, _evict_to_budget
// :2236-2291).  The reference installs in read-completion order
// (:2482-2519); here installs run in ascending expert id so the table is a
// deterministic function of the request sequence.
//
// Prefill fetch groups follow _begin(prefill=True) with PREFILL_TOUCH=0 and
// PREFILL_SLAB=1 (:2347-2453) and install="soft" (_install :2306-2312):
// hits keep their recency and frequency, misses take free slots only (never
// an eviction) and become resident only while the resident count is under
// the budget; the rest of a group's slots (free-list slots it could not
// install, and slots of the prefill stage, ensure_stage :1345-1390) are held
// by the group's ticket and handed back when the group is done
// (_stage_return :1427-1440, _release_slot :1101-1116).
//
// Speculative reads (prediction-driven prefetch: ExpertCache.prefetch
// cache.py:2853, _prefetch_locked with evict_ok=False, staging _raw_ready,
// claim in _begin via _drop_raw :2379-2386) go through a second copy engine
// into free slots only, never evicting.  A staged guess is neither resident
// nor in the table; the fetch of its layer claims it (installed at its slot
// with no new read; the compute stream joins its copy batch, and a claim
// whose copy had not landed yet counts as a miss, as an in-flight read does
// in the reference) and hands back the layer's unclaimed guesses, whose slots
// return to the free list only once their copies have landed.
//
// The device table [layers, experts] int32 (-1 = absent) is the flow table
// (:791-859).  A row is marked dirty whenever its host copy changes (an
// install, an eviction by any layer's fetch, a group's slots coming back),
// and pmoe_slab_sync_table republishes only dirty rows (flow_table :843-859).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "pmoe_internal.h"

namespace {

constexpr int kFreqMax = 8;
constexpr int kPublishChunk = 512;
constexpr int kMaxTickets = 64;
constexpr int kMaxSpecBatches = 64;  // the copy engine's batch records

struct TableChunk {
  int32_t v[kPublishChunk];
};

__global__ void publish_kernel(const TableChunk chunk, int count, int32_t* __restrict__ dst) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) dst[i] = chunk.v[i];
}

// Slots one prefill group holds for its own compute only.
struct Ticket {
  bool live = false;
  int layer = -1;
  std::vector<std::pair<int, int>> temp;  // (expert, slot) not installed as resident
  std::vector<int> from_free, from_stage;
  std::vector<int> claims;                // speculation batches of claimed prefill-ahead reads
};

}  // namespace

struct pmoe_slab {
  int slots = 0, n_layers = 0, n_experts = 0, reserve = 0, budget = 0;
  int lfru = 1, lfru_scan = 8;
  bool stitched = false;
  std::vector<int> free_slots;            // stack; back() is popped first
  // LRU over dense keys (layer*E + e): head = least recent, tail = most recent
  std::vector<int> prev, next, slot_of, freq;
  std::vector<char> in_lru, stitch_key;
  std::vector<char> pending;              // per key: admitted, its copy not yet installed
  int head = -1, tail = -1, lru_size = 0;
  std::vector<char> pinned;               // per routed slot
  std::vector<int> pinned_list;
  std::vector<int32_t> table;             // host [layers*E]
  std::vector<char> dirty;                // per layer: host row not yet published
  int32_t* dtable = nullptr;              // device [layers*E]
  // prefill stage: slab slots [stage_first, stage_first + stage_n)
  int stage_first = 0, stage_n = 0;
  std::vector<int> stage_free;            // stack
  Ticket tickets[kMaxTickets];
  // speculation: staged[key] = slot of a guess whose read was started
  std::vector<int> staged_slot, staged_batch;
  std::vector<int> staged_keys;
  std::vector<std::pair<int, int>> draining;  // (slot, batch) of dropped guesses
  int batch_refs[kMaxSpecBatches] = {};
  pmoe_copy_engine* spec_ce = nullptr;
  std::vector<std::pair<int, int>> claims;    // (key, batch) of the last request
  pmoe_slab_stats st{};
  std::mutex mu;

  void lru_unlink(int k) {
    const int p = prev[k], n = next[k];
    if (p >= 0) next[p] = n; else head = n;
    if (n >= 0) prev[n] = p; else tail = p;
    prev[k] = next[k] = -1;
    in_lru[k] = 0;
    --lru_size;
  }
  void lru_push_back(int k) {
    prev[k] = tail;
    next[k] = -1;
    if (tail >= 0) next[tail] = k; else head = k;
    tail = k;
    in_lru[k] = 1;
    ++lru_size;
  }
  void move_to_end(int k) {
    if (tail == k) return;
    lru_unlink(k);
    lru_push_back(k);
  }
  void set_entry(int k, int32_t slot) {
    table[k] = slot;
    dirty[k / n_experts] = 1;
  }
  void pin(int slot) {
    if (slot >= 0 && !pinned[slot]) {
      pinned[slot] = 1;
      pinned_list.push_back(slot);
    }
  }
  void clear_pins() {
    for (int s : pinned_list) pinned[s] = 0;
    pinned_list.clear();
  }
  bool evictable(int k) const { return !stitch_key[k] && !pinned[slot_of[k]]; }
  void evict(int k) {
    lru_unlink(k);
    freq[k] = 0;
    const int s = slot_of[k];
    slot_of[k] = -1;
    set_entry(k, -1);
    free_slots.push_back(s);
    ++st.evictions;
  }
  int alloc(bool evict_ok) {
    if (!free_slots.empty()) {
      const int s = free_slots.back();
      free_slots.pop_back();
      return s;
    }
    if (!evict_ok) return -1;
    for (int k = head; k >= 0; k = next[k]) {
      if (!evictable(k)) continue;
      evict(k);
      const int s = free_slots.back();
      free_slots.pop_back();
      return s;
    }
    // nothing evictable: give up an unclaimed guess, the latest staged first
    // (cache.py:1149-1157); its read must land before the slot is reused
    // (a guess in a prefill stage slot is never taken for a resident entry)
    for (size_t i = staged_keys.size(); spec_ce && i-- > 0;) {
      const int k = staged_keys[i];
      const int slot = staged_slot[k], b = staged_batch[k];
      if (slot >= slots) continue;
      if (pmoe_copy_batch_wait(spec_ce, b) != PMOE_OK) break;
      staged_slot[k] = -1;
      staged_batch[k] = -1;
      staged_keys.erase(staged_keys.begin() + long(i));
      ++st.spec_dropped;
      if (--batch_refs[b] == 0) (void)pmoe_copy_batch_release(spec_ce, b);
      return slot;
    }
    ++st.starved;
    return -1;
  }
  void install(int k, int slot) {
    slot_of[k] = slot;
    lru_push_back(k);
    set_entry(k, slot);
    ++st.installs;
  }
  void trim() {
    const int scan = lfru ? lfru_scan : 0;
    while (lru_size > budget && lru_size > 1) {
      for (int i = 0; i < scan; ++i) {
        if (lru_size <= 1) break;
        const int k = head;
        if (freq[k] <= 0) break;
        freq[k] >>= 1;
        move_to_end(k);
      }
      int victim = -1;
      for (int k = head; k >= 0; k = next[k])
        if (evictable(k)) {
          victim = k;
          break;
        }
      if (victim < 0) break;
      evict(victim);
    }
  }
  // a guess leaves the staged set; its slot drains back once its read lands
  void drop_staged(int k) {
    draining.emplace_back(staged_slot[k], staged_batch[k]);
    staged_slot[k] = -1;
    staged_batch[k] = -1;
    staged_keys.erase(std::find(staged_keys.begin(), staged_keys.end(), k));
    ++st.spec_dropped;
  }
  void drop_layer_staged(int layer) {
    std::vector<int> keys;
    for (int k : staged_keys)
      if (k / n_experts == layer) keys.push_back(k);
    for (int k : keys) drop_staged(k);
  }
  int live_tickets() const {
    int n = 0;
    for (const Ticket& t : tickets) n += t.live;
    return n;
  }
};

extern "C" int pmoe_slab_create(pmoe_slab** out, int slots, int n_layers, int n_experts,
                                float reserve_frac, int lfru, int lfru_scan) {
  pmoe::clear_error();
  if (!out) return pmoe::fail(PMOE_EINVAL, "slab_create: null out");
  *out = nullptr;
  if (slots <= 0 || n_layers <= 0 || n_experts <= 0)
    return pmoe::fail(PMOE_EINVAL, "slab_create: slots, layers and experts must be positive");
  if (!(reserve_frac >= 0.0f && reserve_frac < 1.0f) || lfru_scan < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_create: bad reserve_frac or lfru_scan");
  auto* s = new (std::nothrow) pmoe_slab();
  if (!s) return pmoe::fail(PMOE_ENOMEM, "slab_create: out of host memory");
  s->slots = slots;
  s->n_layers = n_layers;
  s->n_experts = n_experts;
  s->lfru = lfru ? 1 : 0;
  s->lfru_scan = lfru_scan;
  s->reserve = std::max(4, int(float(slots) * reserve_frac));
  s->budget = slots - s->reserve;
  for (int i = slots - 1; i >= 0; --i) s->free_slots.push_back(i);
  const size_t keys = size_t(n_layers) * n_experts;
  s->prev.assign(keys, -1);
  s->next.assign(keys, -1);
  s->slot_of.assign(keys, -1);
  s->freq.assign(keys, 0);
  s->in_lru.assign(keys, 0);
  s->stitch_key.assign(keys, 0);
  s->pending.assign(keys, 0);
  s->staged_slot.assign(keys, -1);
  s->staged_batch.assign(keys, -1);
  s->pinned.assign(slots, 0);
  s->table.assign(keys, -1);
  s->dirty.assign(n_layers, 0);
  s->st.slots = slots;
  s->st.reserve = s->reserve;
  s->st.budget = s->budget;
  *out = s;
  return PMOE_OK;
}

extern "C" int pmoe_slab_destroy(pmoe_slab* s) {
  pmoe::clear_error();
  if (!s) return PMOE_OK;
  if (s->dtable) (void)hipFree(s->dtable);
  delete s;
  return PMOE_OK;
}

// The device table is allocated on first use (the policy itself never needs
// the GPU) and starts as a copy of the host table.
static int ensure_device_table(pmoe_slab* s) {
  if (s->dtable) return PMOE_OK;
  const size_t bytes = s->table.size() * sizeof(int32_t);
  PMOE_HIP(hipMalloc(reinterpret_cast<void**>(&s->dtable), bytes));
  hipError_t e = hipMemcpy(s->dtable, s->table.data(), bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(s->dtable);
    s->dtable = nullptr;
    return pmoe::hip_fail(e, "slab: device table init");
  }
  std::fill(s->dirty.begin(), s->dirty.end(), 0);
  return PMOE_OK;
}

// Enqueue the upload of one row (its host entries, then the overlay of a
// prefill ticket's temporary slots when one is given).  Caller holds mu.
static int publish_row(pmoe_slab* s, int layer, const Ticket* overlay, hipStream_t st) {
  int rc = ensure_device_table(s);
  if (rc) return rc;
  const int32_t* row = s->table.data() + size_t(layer) * s->n_experts;
  int32_t* dst = s->dtable + size_t(layer) * s->n_experts;
  for (int off = 0; off < s->n_experts; off += kPublishChunk) {
    TableChunk c;
    const int cnt = std::min(kPublishChunk, s->n_experts - off);
    std::copy_n(row + off, cnt, c.v);
    if (overlay)
      for (const auto& es : overlay->temp)
        if (es.first >= off && es.first < off + cnt) c.v[es.first - off] = es.second;
    publish_kernel<<<(cnt + 255) / 256, 256, 0, st>>>(c, cnt, dst + off);
    PMOE_LAUNCH_CHECK("publish_kernel");
    if (pmoe::ledger_on()) {
      if (off == 0) pmoe::ledger_put(PMOE_LEDGER_PUBLISH, s, layer);
      for (int i = 0; i < cnt; ++i)
        if (c.v[i] >= 0) pmoe::ledger_put(PMOE_LEDGER_ROW, s, layer, off + i, c.v[i]);
    }
  }
  s->dirty[layer] = overlay ? 1 : 0;  // an overlay row differs from the host row
  return PMOE_OK;
}

extern "C" const int32_t* pmoe_slab_device_table(pmoe_slab* s, int layer) {
  pmoe::clear_error();
  if (!s || layer < 0 || layer >= s->n_layers) {
    pmoe::set_error("slab_device_table: bad argument");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(s->mu);
  if (ensure_device_table(s)) return nullptr;
  return s->dtable + size_t(layer) * s->n_experts;
}

extern "C" int pmoe_slab_host_table(pmoe_slab* s, int layer, int32_t* out) {
  pmoe::clear_error();
  if (!s || !out || layer < 0 || layer >= s->n_layers)
    return pmoe::fail(PMOE_EINVAL, "slab_host_table: bad argument");
  std::lock_guard<std::mutex> lk(s->mu);
  std::copy_n(s->table.begin() + size_t(layer) * s->n_experts, s->n_experts, out);
  return PMOE_OK;
}

// Sorted distinct ids, each checked against the expert count.
static int unique_ids(pmoe_slab* s, const int32_t* ids, int n_ids, std::vector<int>& uniq,
                      const char* who) {
  uniq.assign(ids, ids + n_ids);
  for (int e : uniq)
    if (e < 0 || e >= s->n_experts)
      return pmoe::fail(PMOE_EINVAL, std::string(who) + ": id out of range");
  std::sort(uniq.begin(), uniq.end());
  uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
  return PMOE_OK;
}

extern "C" int pmoe_slab_request(pmoe_slab* s, int layer, const int32_t* ids, int n_ids,
                                 int32_t* miss_ids, int32_t* miss_slots, int* n_miss) {
  pmoe::clear_error();
  if (!s || (n_ids > 0 && !ids) || !n_miss || layer < 0 || layer >= s->n_layers || n_ids < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_request: bad argument");
  std::vector<int> uniq;
  int rc = unique_ids(s, ids, n_ids, uniq, "slab_request");
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(s->mu);
  const int base = layer * s->n_experts;
  for (int e : uniq)
    if (s->pending[base + e])
      return pmoe::fail(PMOE_EINVAL, "slab_request: an admitted expert's copy is not installed");
  s->clear_pins();
  s->claims.clear();
  std::vector<int> misses;
  std::vector<std::pair<int, int>> claimed;  // (expert, slot): installed with the misses
  for (int e : uniq) {
    const int k = base + e;
    if (s->in_lru[k]) {
      ++s->st.hits;
      s->move_to_end(k);
      s->freq[k] = std::min(kFreqMax, s->freq[k] + 1);
      s->pin(s->slot_of[k]);
    } else if (s->staged_slot[k] >= 0 && s->staged_slot[k] < s->slots) {
      // a guess claimed: no new read (a prefill-ahead read in a stage slot is
      // not made resident there; it is handed back below)
      ++s->st.hits;
      ++s->st.spec_claims;
      const int slot = s->staged_slot[k];
      s->claims.emplace_back(k, s->staged_batch[k]);
      s->staged_slot[k] = -1;
      s->staged_batch[k] = -1;
      s->staged_keys.erase(std::find(s->staged_keys.begin(), s->staged_keys.end(), k));
      s->pin(slot);
      claimed.emplace_back(e, slot);
    } else {
      ++s->st.misses;
      misses.push_back(e);
    }
  }
  int placed = 0;
  std::vector<std::pair<int, int>> got;
  for (int e : misses) {
    const int slot = s->alloc(true);
    if (slot < 0) continue;
    s->pin(slot);
    got.emplace_back(e, slot);
  }
  // installs (claimed guesses and placed misses) in ascending expert id, each
  // followed by the trim, once every entry of this step is pinned
  std::vector<std::pair<int, int>> all(claimed);
  all.insert(all.end(), got.begin(), got.end());
  std::sort(all.begin(), all.end());
  for (auto& es : all) {
    s->install(base + es.first, es.second);
    s->trim();
  }
  for (auto& es : got) {
    if (miss_ids) miss_ids[placed] = es.first;
    if (miss_slots) miss_slots[placed] = es.second;
    ++placed;
  }
  s->drop_layer_staged(layer);  // this layer's guesses it did not route
  *n_miss = placed;
  return PMOE_OK;
}

extern "C" int pmoe_slab_admit(pmoe_slab* s, int layer, const int32_t* ids, int n_ids,
                               int32_t* miss_ids, int32_t* miss_slots, int* n_miss,
                               int clear_pins) {
  pmoe::clear_error();
  if (!s || (n_ids > 0 && !ids) || !n_miss || layer < 0 || layer >= s->n_layers || n_ids < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_admit: bad argument");
  std::vector<int> uniq;
  int rc = unique_ids(s, ids, n_ids, uniq, "slab_admit");
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(s->mu);
  if (clear_pins) s->clear_pins();
  s->drop_layer_staged(layer);
  const int base = layer * s->n_experts;
  int placed = 0;
  for (int e : uniq) {
    const int k = base + e;
    if (s->in_lru[k]) {
      ++s->st.hits;
      s->move_to_end(k);
      s->freq[k] = std::min(kFreqMax, s->freq[k] + 1);
      continue;
    }
    ++s->st.misses;
    if (s->pending[k]) continue;  // its read is already in flight
    const int slot = s->alloc(true);
    if (slot < 0) break;          // nothing evictable: admit no more of this layer
    s->pending[k] = 1;
    s->slot_of[k] = slot;
    ++s->st.flow_admits;
    if (miss_ids) miss_ids[placed] = e;
    if (miss_slots) miss_slots[placed] = slot;
    ++placed;
  }
  *n_miss = placed;
  return PMOE_OK;
}

extern "C" int pmoe_slab_install(pmoe_slab* s, int layer, const int32_t* ids, int n_ids) {
  pmoe::clear_error();
  if (!s || (n_ids > 0 && !ids) || layer < 0 || layer >= s->n_layers || n_ids < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_install: bad argument");
  std::vector<int> uniq;
  int rc = unique_ids(s, ids, n_ids, uniq, "slab_install");
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(s->mu);
  const int base = layer * s->n_experts;
  for (int e : uniq)
    if (!s->pending[base + e])
      return pmoe::fail(PMOE_EINVAL, "slab_install: expert was not admitted");
  for (int e : uniq) {
    const int k = base + e;
    s->pending[k] = 0;
    s->install(k, s->slot_of[k]);
    s->trim();
  }
  return PMOE_OK;
}

extern "C" int pmoe_slab_set_spec_engine(pmoe_slab* s, pmoe_copy_engine* ce) {
  pmoe::clear_error();
  if (!s) return pmoe::fail(PMOE_EINVAL, "slab_set_spec_engine: null slab");
  std::lock_guard<std::mutex> lk(s->mu);
  if (!s->staged_keys.empty() || !s->draining.empty())
    return pmoe::fail(PMOE_EINVAL, "slab_set_spec_engine: speculative reads outstanding");
  s->spec_ce = ce;
  return PMOE_OK;
}

// Caller holds mu.  Dropped guesses whose reads have landed give back their
// slots; batch records nothing references any more are released.
static int settle_spec(pmoe_slab* s) {
  if (!s->spec_ce) return PMOE_OK;
  std::vector<std::pair<int, int>> keep;
  for (auto& sb : s->draining) {
    const int r = pmoe_copy_batch_done(s->spec_ce, sb.second);
    if (r < 0) return r;
    if (r == 0) {
      keep.push_back(sb);
      continue;
    }
    if (sb.first >= s->slots)
      s->stage_free.push_back(sb.first);
    else
      s->free_slots.push_back(sb.first);
    if (--s->batch_refs[sb.second] == 0) {
      const int rc = pmoe_copy_batch_release(s->spec_ce, sb.second);
      if (rc) return rc;
    }
  }
  s->draining.swap(keep);
  return PMOE_OK;
}

extern "C" int pmoe_slab_speculate(pmoe_slab* s, const pmoe_geom* g, void* slab,
                                   const void* host_store, int layer, const int32_t* ids,
                                   int n_ids, int max_staged, int* n_started) {
  pmoe::clear_error();
  if (!s || !g || !slab || !host_store || (n_ids > 0 && !ids) || !n_started || layer < 0 ||
      layer >= s->n_layers || n_ids < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_speculate: bad argument");
  *n_started = 0;
  std::lock_guard<std::mutex> lk(s->mu);
  if (!s->spec_ce) return pmoe::fail(PMOE_EINVAL, "slab_speculate: no speculation engine");
  int rc = settle_spec(s);
  if (rc) return rc;
  const int base = layer * s->n_experts;
  std::vector<std::pair<int, int>> got;  // (key, slot)
  for (int i = 0; i < n_ids; ++i) {
    const int e = ids[i];
    if (e < 0 || e >= s->n_experts) return pmoe::fail(PMOE_EINVAL, "slab_speculate: id out of range");
    const int k = base + e;
    if (s->in_lru[k] || s->pending[k] || s->staged_slot[k] >= 0) continue;
    bool dup = false;
    for (auto& ks : got) dup |= ks.first == k;
    if (dup) continue;
    if (int(s->staged_keys.size() + got.size()) >= max_staged || s->free_slots.empty()) break;
    // every outstanding guess holds one of the engine's batch records
    if (int(s->staged_keys.size() + s->draining.size() + got.size()) >= kMaxSpecBatches - 1) break;
    got.emplace_back(k, s->free_slots.back());
    s->free_slots.pop_back();
  }
  if (got.empty()) return PMOE_OK;
  // one copy batch per guess: a claim waits for its own read only
  const size_t eb = size_t(g->expert_bytes);
  size_t started = 0;
  for (; started < got.size(); ++started) {
    const auto& ks = got[started];
    rc = pmoe_copy_submit(s->spec_ce, static_cast<uint8_t*>(slab) + size_t(ks.second) * eb,
                          static_cast<const uint8_t*>(host_store) + size_t(ks.first) * eb, eb, 0);
    int b = -1;
    if (!rc) rc = pmoe_copy_issue(s->spec_ce, &b);
    if (rc) break;
    s->staged_slot[ks.first] = ks.second;
    s->staged_batch[ks.first] = b;
    s->staged_keys.push_back(ks.first);
    s->batch_refs[b] = 1;
  }
  for (size_t i = got.size(); i-- > started;) s->free_slots.push_back(got[i].second);
  s->st.spec_started += int64_t(started);
  s->st.bytes_copied += int64_t(started) * int64_t(eb);
  *n_started = int(started);
  if (rc && started == 0) return rc;
  pmoe::clear_error();  // a guess that could not start is not an error of the call
  return PMOE_OK;
}

extern "C" int pmoe_slab_prefill_ahead(pmoe_slab* s, const pmoe_geom* g, void* slab,
                                       const void* host_store, int layer, const int32_t* ids,
                                       int n_ids, int free_floor, int stage_floor,
                                       int* n_started) {
  pmoe::clear_error();
  if (!s || !g || !slab || !host_store || (n_ids > 0 && !ids) || !n_started || layer < 0 ||
      layer >= s->n_layers || n_ids < 0 || free_floor < 0 || stage_floor < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_prefill_ahead: bad argument");
  *n_started = 0;
  std::lock_guard<std::mutex> lk(s->mu);
  if (!s->spec_ce) return pmoe::fail(PMOE_EINVAL, "slab_prefill_ahead: no speculation engine");
  int rc = settle_spec(s);
  if (rc) return rc;
  const int base = layer * s->n_experts;
  std::vector<std::pair<int, int>> got;  // (key, slot)
  std::vector<char> seen(size_t(s->n_experts), 0);
  for (int i = 0; i < n_ids; ++i) {
    const int e = ids[i];
    if (e < 0 || e >= s->n_experts) return pmoe::fail(PMOE_EINVAL, "slab_prefill_ahead: id out of range");
    const int k = base + e;
    if (seen[e] || s->in_lru[k] || s->pending[k] || s->staged_slot[k] >= 0) continue;
    seen[e] = 1;
    int slot = -1;
    if (int(s->free_slots.size()) > free_floor) {
      slot = s->free_slots.back();
      s->free_slots.pop_back();
    } else if (int(s->stage_free.size()) > stage_floor) {
      slot = s->stage_free.back();
      s->stage_free.pop_back();
    } else {
      break;
    }
    got.emplace_back(k, slot);
  }
  if (got.empty()) return PMOE_OK;
  // one copy batch for the whole set: the next layer's groups want most of it
  const size_t eb = size_t(g->expert_bytes);
  for (const auto& ks : got) {
    rc = pmoe_copy_submit(s->spec_ce, static_cast<uint8_t*>(slab) + size_t(ks.second) * eb,
                          static_cast<const uint8_t*>(host_store) + size_t(ks.first) * eb, eb, 0);
    if (rc) break;
  }
  int b = -1;
  if (!rc) rc = pmoe_copy_issue(s->spec_ce, &b);
  if (rc) {  // nothing was issued: the slots go back where they came from
    for (size_t i = got.size(); i-- > 0;)
      (got[i].second >= s->slots ? s->stage_free : s->free_slots).push_back(got[i].second);
    return rc;
  }
  for (const auto& ks : got) {
    s->staged_slot[ks.first] = ks.second;
    s->staged_batch[ks.first] = b;
    s->staged_keys.push_back(ks.first);
  }
  s->batch_refs[b] = int(got.size());
  s->st.ahead_started += int64_t(got.size());
  s->st.bytes_copied += int64_t(got.size()) * int64_t(eb);
  *n_started = int(got.size());
  return PMOE_OK;
}

extern "C" int pmoe_slab_drop_staged(pmoe_slab* s) {
  pmoe::clear_error();
  if (!s) return pmoe::fail(PMOE_EINVAL, "slab_drop_staged: null slab");
  std::lock_guard<std::mutex> lk(s->mu);
  while (!s->staged_keys.empty()) s->drop_staged(s->staged_keys.back());
  return settle_spec(s);
}

extern "C" int pmoe_slab_set_stage(pmoe_slab* s, int first_slot, int n_slots) {
  pmoe::clear_error();
  if (!s || n_slots < 0 || (n_slots > 0 && first_slot < s->slots))
    return pmoe::fail(PMOE_EINVAL, "slab_set_stage: stage slots must follow the routed slots");
  std::lock_guard<std::mutex> lk(s->mu);
  if (s->live_tickets())
    return pmoe::fail(PMOE_EINVAL, "slab_set_stage: a prefill group still holds stage slots");
  s->stage_first = first_slot;
  s->stage_n = n_slots;
  s->stage_free.clear();
  for (int i = n_slots - 1; i >= 0; --i) s->stage_free.push_back(first_slot + i);
  return PMOE_OK;
}

extern "C" int pmoe_slab_capacity(pmoe_slab* s, int* free_slots, int* stage_free,
                                  int* budget_room) {
  pmoe::clear_error();
  if (!s) return pmoe::fail(PMOE_EINVAL, "slab_capacity: null slab");
  std::lock_guard<std::mutex> lk(s->mu);
  if (free_slots) *free_slots = int(s->free_slots.size());
  if (stage_free) *stage_free = int(s->stage_free.size());
  if (budget_room) *budget_room = std::max(0, s->budget - s->lru_size);
  return PMOE_OK;
}

extern "C" int pmoe_slab_prefill_request(pmoe_slab* s, int layer, const int32_t* ids, int n_ids,
                                         int32_t* miss_ids, int32_t* miss_slots, int* n_miss,
                                         int* n_unplaced, int* ticket) {
  pmoe::clear_error();
  if (!s || (n_ids > 0 && !ids) || !n_miss || !ticket || layer < 0 || layer >= s->n_layers ||
      n_ids < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_prefill_request: bad argument");
  std::vector<int> uniq;
  int rc = unique_ids(s, ids, n_ids, uniq, "slab_prefill_request");
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(s->mu);
  int t = -1;
  for (int i = 0; i < kMaxTickets && t < 0; ++i)
    if (!s->tickets[i].live) t = i;
  if (t < 0) return pmoe::fail(PMOE_EINVAL, "slab_prefill_request: too many open prefill groups");
  const int base = layer * s->n_experts;
  for (int e : uniq)
    if (s->pending[base + e])
      return pmoe::fail(PMOE_EINVAL,
                        "slab_prefill_request: an admitted expert's copy is not installed");
  Ticket& tk = s->tickets[t];
  tk = Ticket();
  tk.live = true;
  tk.layer = layer;
  int placed = 0, unplaced = 0;
  for (int e : uniq) {
    const int k = base + e;
    if (s->in_lru[k]) {  // hit: recency and frequency untouched
      ++s->st.hits;
      continue;
    }
    if (s->staged_slot[k] >= 0) {  // a prefill-ahead read already issued: claimed
      const int slot = s->staged_slot[k];
      tk.claims.push_back(s->staged_batch[k]);
      s->staged_slot[k] = -1;
      s->staged_batch[k] = -1;
      s->staged_keys.erase(std::find(s->staged_keys.begin(), s->staged_keys.end(), k));
      ++s->st.hits;
      ++s->st.ahead_claims;
      if (slot < s->slots && s->lru_size < s->budget) {
        s->install(k, slot);
        ++s->st.prefill_installs;
      } else {
        tk.temp.emplace_back(e, slot);
        (slot < s->slots ? tk.from_free : tk.from_stage).push_back(slot);
      }
      continue;
    }
    ++s->st.misses;
    int slot = s->alloc(false);
    if (slot >= 0) {
      ++s->st.prefill_slot_reads;
      if (s->lru_size < s->budget) {  // soft install: only into room under the budget
        s->install(k, slot);
        ++s->st.prefill_installs;
      } else {
        tk.temp.emplace_back(e, slot);
        tk.from_free.push_back(slot);
      }
    } else if (!s->stage_free.empty()) {
      slot = s->stage_free.back();
      s->stage_free.pop_back();
      tk.temp.emplace_back(e, slot);
      tk.from_stage.push_back(slot);
      ++s->st.stage_reads;
    } else {
      ++s->st.prefill_starved;
      ++unplaced;
      continue;
    }
    if (miss_ids) miss_ids[placed] = e;
    if (miss_slots) miss_slots[placed] = slot;
    ++placed;
  }
  s->drop_layer_staged(layer);  // this layer's guesses it did not route
  *n_miss = placed;
  if (n_unplaced) *n_unplaced = unplaced;
  *ticket = t;
  return PMOE_OK;
}

static Ticket* live_ticket(pmoe_slab* s, int ticket) {
  if (ticket < 0 || ticket >= kMaxTickets || !s->tickets[ticket].live) return nullptr;
  return &s->tickets[ticket];
}

extern "C" int pmoe_slab_prefill_publish(pmoe_slab* s, int ticket, void* stream) {
  pmoe::clear_error();
  if (!s) return pmoe::fail(PMOE_EINVAL, "slab_prefill_publish: null slab");
  std::lock_guard<std::mutex> lk(s->mu);
  Ticket* tk = live_ticket(s, ticket);
  if (!tk) return pmoe::fail(PMOE_EINVAL, "slab_prefill_publish: no such open prefill group");
  // the group computes on claimed prefill-ahead reads: wait for their batches
  for (int b : tk->claims) {
    int rc = pmoe_copy_batch_join(s->spec_ce, b, stream);
    if (!rc && --s->batch_refs[b] == 0) rc = pmoe_copy_batch_release(s->spec_ce, b);
    if (rc) return rc;
  }
  tk->claims.clear();
  return publish_row(s, tk->layer, tk, static_cast<hipStream_t>(stream));
}

extern "C" int pmoe_slab_prefill_done(pmoe_slab* s, int ticket) {
  pmoe::clear_error();
  if (!s) return pmoe::fail(PMOE_EINVAL, "slab_prefill_done: null slab");
  std::lock_guard<std::mutex> lk(s->mu);
  Ticket* tk = live_ticket(s, ticket);
  if (!tk) return pmoe::fail(PMOE_EINVAL, "slab_prefill_done: no such open prefill group");
  for (int b : tk->claims)  // never published: the host waits for those reads
    if (pmoe_copy_batch_wait(s->spec_ce, b) == PMOE_OK && --s->batch_refs[b] == 0)
      (void)pmoe_copy_batch_release(s->spec_ce, b);
  for (int slot : tk->from_free) s->free_slots.push_back(slot);
  for (int slot : tk->from_stage) s->stage_free.push_back(slot);
  if (!tk->temp.empty()) s->dirty[tk->layer] = 1;
  *tk = Ticket();
  return PMOE_OK;
}

extern "C" int pmoe_slab_stitch(pmoe_slab* s) {
  pmoe::clear_error();
  if (!s) return pmoe::fail(PMOE_EINVAL, "slab_stitch: null slab");
  std::lock_guard<std::mutex> lk(s->mu);
  if (s->stitched) return 1;
  const long total = long(s->n_layers) * s->n_experts;
  if (total > s->slots) return 0;
  for (int k = 0; k < total; ++k) {
    if (s->in_lru[k]) continue;
    const int slot = s->alloc(false);
    if (slot < 0) return 0;
    s->install(k, slot);
    --s->st.installs;  // a stitch load is not a demand install
  }
  for (int k = 0; k < total; ++k) s->stitch_key[k] = 1;
  s->budget = s->slots;
  s->st.budget = s->budget;
  s->stitched = true;
  return 1;
}

extern "C" int pmoe_slab_publish(pmoe_slab* s, int layer, void* stream) {
  pmoe::clear_error();
  if (!s || layer < 0 || layer >= s->n_layers)
    return pmoe::fail(PMOE_EINVAL, "slab_publish: bad argument");
  std::lock_guard<std::mutex> lk(s->mu);
  return publish_row(s, layer, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int pmoe_slab_sync_table(pmoe_slab* s, int layer, void* stream) {
  pmoe::clear_error();
  if (!s || layer < 0 || layer >= s->n_layers)
    return pmoe::fail(PMOE_EINVAL, "slab_sync_table: bad argument");
  std::lock_guard<std::mutex> lk(s->mu);
  if (s->dtable && !s->dirty[layer]) return 0;
  const int rc = publish_row(s, layer, nullptr, static_cast<hipStream_t>(stream));
  return rc ? rc : 1;
}

extern "C" int pmoe_slab_read_device_row(pmoe_slab* s, int layer, int32_t* out) {
  pmoe::clear_error();
  if (!s || !out || layer < 0 || layer >= s->n_layers)
    return pmoe::fail(PMOE_EINVAL, "slab_read_device_row: bad argument");
  int32_t* src = nullptr;
  {
    std::lock_guard<std::mutex> lk(s->mu);
    int rc = ensure_device_table(s);
    if (rc) return rc;
    src = s->dtable + size_t(layer) * s->n_experts;
  }
  PMOE_HIP(hipDeviceSynchronize());
  PMOE_HIP(hipMemcpy(out, src, size_t(s->n_experts) * sizeof(int32_t), hipMemcpyDeviceToHost));
  return PMOE_OK;
}

extern "C" int pmoe_slab_dirty(pmoe_slab* s, int layer) {
  pmoe::clear_error();
  if (!s || layer < 0 || layer >= s->n_layers)
    return pmoe::fail(PMOE_EINVAL, "slab_dirty: bad argument");
  std::lock_guard<std::mutex> lk(s->mu);
  return s->dirty[layer] ? 1 : 0;
}

extern "C" int pmoe_slab_stats_get(pmoe_slab* s, pmoe_slab_stats* out) {
  pmoe::clear_error();
  if (!s || !out) return pmoe::fail(PMOE_EINVAL, "slab_stats: bad argument");
  std::lock_guard<std::mutex> lk(s->mu);
  s->st.resident = s->lru_size;
  s->st.stitched = s->stitched ? 1 : 0;
  s->st.stage_slots = s->stage_n;
  *out = s->st;
  return PMOE_OK;
}

// Copy the placed misses of one request from the host store into the slab.
static int submit_misses(pmoe_slab* s, pmoe_copy_engine* ce, const pmoe_geom* g, void* slab,
                         const void* host_store, int layer, const int32_t* mid,
                         const int32_t* msl, int nm) {
  const size_t eb = size_t(g->expert_bytes);
  for (int i = 0; i < nm; ++i) {
    const size_t src = (size_t(layer) * s->n_experts + size_t(mid[i])) * eb;
    const int rc = pmoe_copy_submit(ce, static_cast<uint8_t*>(slab) + size_t(msl[i]) * eb,
                                    static_cast<const uint8_t*>(host_store) + src, eb, 1);
    if (rc) return rc;
  }
  std::lock_guard<std::mutex> lk(s->mu);
  s->st.bytes_copied += int64_t(nm) * int64_t(eb);
  return PMOE_OK;
}

extern "C" int pmoe_slab_fetch(pmoe_slab* s, pmoe_copy_engine* ce, const pmoe_geom* g,
                               void* slab, const void* host_store, int layer, const int32_t* ids,
                               int n_ids, int* n_miss, void* stream) {
  pmoe::clear_error();
  if (!s || !ce || !g || !slab || !host_store || !n_miss || n_ids < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_fetch: bad argument");
  std::vector<int32_t> mid(size_t(n_ids) + 1), msl(size_t(n_ids) + 1);
  int nm = 0;
  int rc;
  {
    std::lock_guard<std::mutex> lk(s->mu);
    rc = settle_spec(s);
  }
  if (rc) return rc;
  rc = pmoe_slab_request(s, layer, ids, n_ids, mid.data(), msl.data(), &nm);
  if (rc) return rc;
  {
    // claimed guesses: the compute stream waits for their reads; one that
    // had not landed counts as a miss (cache.py:2387-2401)
    std::lock_guard<std::mutex> lk(s->mu);
    for (auto& kb : s->claims) {
      const int done = pmoe_copy_batch_done(s->spec_ce, kb.second);
      if (done < 0) return done;
      if (!done) {
        --s->st.hits;
        ++s->st.misses;
        ++s->st.spec_claims_late;
      }
      rc = pmoe_copy_batch_join(s->spec_ce, kb.second, stream);
      if (rc) return rc;
      if (--s->batch_refs[kb.second] == 0) {
        rc = pmoe_copy_batch_release(s->spec_ce, kb.second);
        if (rc) return rc;
      }
    }
    s->claims.clear();
  }
  rc = submit_misses(s, ce, g, slab, host_store, layer, mid.data(), msl.data(), nm);
  if (rc) return rc;
  rc = pmoe_slab_publish(s, layer, stream);
  if (rc) return rc;
  rc = pmoe_copy_flush(ce, stream);
  if (rc) return rc;
  *n_miss = nm;
  return PMOE_OK;
}

extern "C" int pmoe_slab_fetch_prefill(pmoe_slab* s, pmoe_copy_engine* ce, const pmoe_geom* g,
                                       void* slab, const void* host_store, int layer,
                                       const int32_t* ids, int n_ids, int* n_miss,
                                       int* n_unplaced, int* ticket) {
  pmoe::clear_error();
  if (!s || !ce || !g || !slab || !host_store || !n_miss || !ticket || n_ids < 0)
    return pmoe::fail(PMOE_EINVAL, "slab_fetch_prefill: bad argument");
  std::vector<int32_t> mid(size_t(n_ids) + 1), msl(size_t(n_ids) + 1);
  int nm = 0, nu = 0, t = -1;
  int rc = pmoe_slab_prefill_request(s, layer, ids, n_ids, mid.data(), msl.data(), &nm, &nu, &t);
  if (rc) return rc;
  rc = submit_misses(s, ce, g, slab, host_store, layer, mid.data(), msl.data(), nm);
  if (!rc) rc = pmoe_copy_issue(ce, nullptr);
  if (rc) {
    (void)pmoe_slab_prefill_done(s, t);
    return rc;
  }
  *n_miss = nm;
  if (n_unplaced) *n_unplaced = nu;
  *ticket = t;
  return PMOE_OK;
}
