// Host -> HBM copy engine for slab misses.
//
// Counterpart of the reference's native read pool (_native_read.c:38-698):
// jobs wait in an urgent and a normal queue (urgent = a layer is blocked on
// it, :260-269), are cut into pieces of at most split_bytes so several copy
// streams / SDMA engines share one expert (:213-241), and the first error of
// a batch is the one reported (:131-156, :293-302).  Instead of pread into
// unified memory, a piece is one hipMemcpyAsync from pinned host memory into
// its slab slot.  Ordering with compute uses events only.  A fence is an
// event recorded on the compute stream; issued copies first wait for the
// latest fence, so no slot is overwritten while a kernel queued before the
// fence may still read it.  A join makes a stream wait for every issued copy.
// pmoe_copy_flush is fence at the stream's tail + issue + join, the decode
// fetch's ordering.  A prefill fetch group fences before the previous group's
// compute and joins only before its own, so its copies run under that
// compute (cache.py:2535-2578: "While group i computes on the GPU, the reads
// for group i+1 are already in flight").  All streams have default priority.
#include <hip/hip_runtime.h>

#include <atomic>
#include <deque>
#include <mutex>
#include <vector>

#include "pmoe_internal.h"

constexpr int kMaxBatches = 64;

// ---------------------------------------------------------------- ledger
// The slot-safety log: one vector for the process, in call order, capped so
// a forgotten drain cannot grow without bound (drops are counted).
namespace {
constexpr size_t kLedgerCap = size_t(1) << 22;
std::atomic<bool> g_ledger_on{false};
std::mutex g_ledger_mu;
std::vector<pmoe_ledger_rec> g_ledger;
int64_t g_ledger_dropped = 0;
}  // namespace

namespace pmoe {
bool ledger_on() { return g_ledger_on.load(std::memory_order_relaxed); }
void ledger_put(int64_t kind, const void* who, int64_t a, int64_t b, int64_t c) {
  if (!ledger_on()) return;
  std::lock_guard<std::mutex> lk(g_ledger_mu);
  if (g_ledger.size() >= kLedgerCap) {
    ++g_ledger_dropped;
    return;
  }
  g_ledger.push_back({kind, int64_t(reinterpret_cast<uintptr_t>(who)), a, b, c});
}
}  // namespace pmoe

extern "C" int pmoe_ledger_enable(int on) {
  pmoe::clear_error();
  std::lock_guard<std::mutex> lk(g_ledger_mu);
  g_ledger.clear();
  g_ledger_dropped = 0;
  g_ledger_on.store(on != 0);
  return PMOE_OK;
}

extern "C" int pmoe_ledger_note(int64_t kind, const void* who, int64_t a, int64_t b, int64_t c) {
  pmoe::clear_error();
  if (kind != PMOE_LEDGER_COMPUTE) return pmoe::fail(PMOE_EINVAL, "ledger_note: caller events are COMPUTE");
  pmoe::ledger_put(kind, who, a, b, c);
  return PMOE_OK;
}

extern "C" int pmoe_ledger_drain(pmoe_ledger_rec* out, int cap, int* n) {
  pmoe::clear_error();
  if (!n || cap < 0 || (cap > 0 && !out)) return pmoe::fail(PMOE_EINVAL, "ledger_drain: bad argument");
  std::lock_guard<std::mutex> lk(g_ledger_mu);
  const size_t take = std::min(g_ledger.size(), size_t(cap));
  std::copy_n(g_ledger.begin(), take, out);
  g_ledger.erase(g_ledger.begin(), g_ledger.begin() + take);
  *n = int(take);
  const int64_t dropped = g_ledger_dropped;
  g_ledger_dropped = 0;
  return int(std::min<int64_t>(dropped, 1 << 30));
}

struct pmoe_copy_engine {
  struct Job {
    void* dst;
    const void* src;
    size_t bytes;
  };
  // An issued set of copies whose completion is tracked on its own: one
  // event per copy stream, recorded right after the batch's copies.
  struct Batch {
    bool live = false;
    std::vector<hipEvent_t> ev;
  };
  Batch batches[kMaxBatches];
  size_t split = size_t(64) << 20;  // whole experts: larger pieces copy faster
  std::vector<hipStream_t> streams;
  std::vector<hipEvent_t> done;
  hipEvent_t fence = nullptr;
  bool fenced = false;
  std::deque<Job> urgent, normal;
  int64_t bytes = 0;
  int next_stream = 0;
  std::mutex mu;
};

extern "C" int pmoe_host_alloc(void** out, size_t bytes) {
  pmoe::clear_error();
  if (!out) return pmoe::fail(PMOE_EINVAL, "host_alloc: null out");
  *out = nullptr;
  if (bytes == 0) return PMOE_OK;
  hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    *out = nullptr;
    return pmoe::fail(PMOE_ENOMEM, std::string("host_alloc: ") + hipGetErrorString(e));
  }
  return PMOE_OK;
}

extern "C" int pmoe_host_free(void* p) {
  pmoe::clear_error();
  if (p) PMOE_HIP(hipHostFree(p));
  return PMOE_OK;
}

extern "C" int pmoe_copy_engine_create(pmoe_copy_engine** out, size_t split_bytes,
                                       int n_streams) {
  pmoe::clear_error();
  if (!out) return pmoe::fail(PMOE_EINVAL, "copy_engine_create: null out");
  *out = nullptr;
  if (n_streams <= 0 || n_streams > 8)
    return pmoe::fail(PMOE_EINVAL, "copy_engine_create: n_streams must be 1..8");
  auto* ce = new (std::nothrow) pmoe_copy_engine();
  if (!ce) return pmoe::fail(PMOE_ENOMEM, "copy_engine_create: out of host memory");
  if (split_bytes > 0) ce->split = split_bytes;
  hipError_t e = hipEventCreateWithFlags(&ce->fence, hipEventDisableTiming);
  for (int i = 0; i < n_streams && e == hipSuccess; ++i) {
    hipStream_t s = nullptr;
    hipEvent_t ev = nullptr;
    e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) ce->streams.push_back(s);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) ce->done.push_back(ev);
  }
  for (int b = 0; b < kMaxBatches && e == hipSuccess; ++b)
    for (int i = 0; i < n_streams && e == hipSuccess; ++i) {
      hipEvent_t ev = nullptr;
      e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (e == hipSuccess) ce->batches[b].ev.push_back(ev);
    }
  if (e != hipSuccess) {
    pmoe_copy_engine_destroy(ce);
    return pmoe::hip_fail(e, "copy_engine_create");
  }
  *out = ce;
  return PMOE_OK;
}

extern "C" int pmoe_copy_engine_destroy(pmoe_copy_engine* ce) {
  pmoe::clear_error();
  if (!ce) return PMOE_OK;
  for (hipStream_t s : ce->streams) {
    (void)hipStreamSynchronize(s);
    (void)hipStreamDestroy(s);
  }
  for (hipEvent_t ev : ce->done) (void)hipEventDestroy(ev);
  for (auto& b : ce->batches)
    for (hipEvent_t ev : b.ev) (void)hipEventDestroy(ev);
  if (ce->fence) (void)hipEventDestroy(ce->fence);
  delete ce;
  return PMOE_OK;
}

extern "C" int pmoe_copy_submit(pmoe_copy_engine* ce, void* dst, const void* src, size_t bytes,
                                int urgent) {
  pmoe::clear_error();
  if (!ce || (bytes && (!dst || !src))) return pmoe::fail(PMOE_EINVAL, "copy_submit: bad argument");
  if (!bytes) return PMOE_OK;
  std::lock_guard<std::mutex> lk(ce->mu);
  (urgent ? ce->urgent : ce->normal).push_back({dst, src, bytes});
  pmoe::ledger_put(PMOE_LEDGER_SUBMIT, ce, int64_t(reinterpret_cast<uintptr_t>(dst)),
                   int64_t(reinterpret_cast<uintptr_t>(src)), int64_t(bytes));
  return PMOE_OK;
}

extern "C" int pmoe_copy_fence(pmoe_copy_engine* ce, void* stream) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_fence: null engine");
  std::lock_guard<std::mutex> lk(ce->mu);
  PMOE_HIP(hipEventRecord(ce->fence, static_cast<hipStream_t>(stream)));
  ce->fenced = true;
  pmoe::ledger_put(PMOE_LEDGER_FENCE, ce);
  return PMOE_OK;
}

// Caller holds mu.  batch: the batch record the copies form (-1: none),
// for the ledger.
static int issue_locked(pmoe_copy_engine* ce, int batch) {
  if (ce->urgent.empty() && ce->normal.empty()) return PMOE_OK;
  pmoe::ledger_put(PMOE_LEDGER_ISSUE, ce, batch);
  if (ce->fenced)
    for (hipStream_t s : ce->streams) PMOE_HIP(hipStreamWaitEvent(s, ce->fence, 0));
  int first_err = PMOE_OK;
  auto issue = [&](std::deque<pmoe_copy_engine::Job>& q) {
    while (!q.empty()) {
      const auto job = q.front();
      q.pop_front();
      for (size_t off = 0; off < job.bytes; off += ce->split) {
        const size_t len = std::min(ce->split, job.bytes - off);
        hipStream_t s = ce->streams[ce->next_stream];
        ce->next_stream = (ce->next_stream + 1) % int(ce->streams.size());
        hipError_t e = hipMemcpyAsync(static_cast<uint8_t*>(job.dst) + off,
                                      static_cast<const uint8_t*>(job.src) + off, len,
                                      hipMemcpyHostToDevice, s);
        if (e != hipSuccess && first_err == PMOE_OK)
          first_err = pmoe::hip_fail(e, "copy_issue: hipMemcpyAsync");
        else if (e == hipSuccess)
          ce->bytes += int64_t(len);
      }
    }
  };
  issue(ce->urgent);
  issue(ce->normal);
  for (size_t i = 0; i < ce->streams.size(); ++i)
    PMOE_HIP(hipEventRecord(ce->done[i], ce->streams[i]));
  return first_err;
}

extern "C" int pmoe_copy_issue(pmoe_copy_engine* ce, int* batch) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_issue: null engine");
  std::lock_guard<std::mutex> lk(ce->mu);
  int b = -1;
  if (batch) {
    for (int i = 0; i < kMaxBatches && b < 0; ++i)
      if (!ce->batches[i].live) b = i;
    if (b < 0) return pmoe::fail(PMOE_EINVAL, "copy_issue: every batch record is in use");
  }
  const int rc = issue_locked(ce, b);
  if (rc) return rc;
  if (batch) {
    for (size_t i = 0; i < ce->streams.size(); ++i)
      PMOE_HIP(hipEventRecord(ce->batches[b].ev[i], ce->streams[i]));
    ce->batches[b].live = true;
    *batch = b;
  }
  return PMOE_OK;
}

static pmoe_copy_engine::Batch* live_batch(pmoe_copy_engine* ce, int b) {
  if (!ce || b < 0 || b >= kMaxBatches || !ce->batches[b].live) return nullptr;
  return &ce->batches[b];
}

extern "C" int pmoe_copy_batch_done(pmoe_copy_engine* ce, int batch) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_batch_done: null engine");
  std::lock_guard<std::mutex> lk(ce->mu);
  auto* b = live_batch(ce, batch);
  if (!b) return pmoe::fail(PMOE_EINVAL, "copy_batch_done: no such batch");
  for (hipEvent_t ev : b->ev) {
    const hipError_t e = hipEventQuery(ev);
    if (e == hipErrorNotReady) return 0;
    if (e != hipSuccess) return pmoe::hip_fail(e, "copy_batch_done: hipEventQuery");
  }
  pmoe::ledger_put(PMOE_LEDGER_HOST_DONE, ce, batch);
  return 1;
}

extern "C" int pmoe_copy_batch_join(pmoe_copy_engine* ce, int batch, void* stream) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_batch_join: null engine");
  std::lock_guard<std::mutex> lk(ce->mu);
  auto* b = live_batch(ce, batch);
  if (!b) return pmoe::fail(PMOE_EINVAL, "copy_batch_join: no such batch");
  for (hipEvent_t ev : b->ev) PMOE_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), ev, 0));
  pmoe::ledger_put(PMOE_LEDGER_BATCH_JOIN, ce, batch);
  return PMOE_OK;
}

extern "C" int pmoe_copy_batch_wait(pmoe_copy_engine* ce, int batch) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_batch_wait: null engine");
  std::vector<hipEvent_t> evs;
  {
    std::lock_guard<std::mutex> lk(ce->mu);
    auto* b = live_batch(ce, batch);
    if (!b) return pmoe::fail(PMOE_EINVAL, "copy_batch_wait: no such batch");
    evs = b->ev;
  }
  for (hipEvent_t ev : evs) PMOE_HIP(hipEventSynchronize(ev));
  pmoe::ledger_put(PMOE_LEDGER_HOST_DONE, ce, batch);
  return PMOE_OK;
}

extern "C" int pmoe_copy_batch_release(pmoe_copy_engine* ce, int batch) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_batch_release: null engine");
  std::lock_guard<std::mutex> lk(ce->mu);
  auto* b = live_batch(ce, batch);
  if (!b) return pmoe::fail(PMOE_EINVAL, "copy_batch_release: no such batch");
  b->live = false;
  return PMOE_OK;
}

extern "C" int pmoe_copy_join(pmoe_copy_engine* ce, void* stream) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_join: null engine");
  std::lock_guard<std::mutex> lk(ce->mu);
  for (hipEvent_t ev : ce->done)
    PMOE_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), ev, 0));
  pmoe::ledger_put(PMOE_LEDGER_JOIN, ce);
  return PMOE_OK;
}

extern "C" int pmoe_copy_flush(pmoe_copy_engine* ce, void* stream) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_flush: null engine");
  hipStream_t compute = static_cast<hipStream_t>(stream);
  std::lock_guard<std::mutex> lk(ce->mu);
  if (ce->urgent.empty() && ce->normal.empty()) return PMOE_OK;
  PMOE_HIP(hipEventRecord(ce->fence, compute));
  ce->fenced = true;
  pmoe::ledger_put(PMOE_LEDGER_FENCE, ce);
  const int rc = issue_locked(ce, -1);
  for (hipEvent_t ev : ce->done) PMOE_HIP(hipStreamWaitEvent(compute, ev, 0));
  pmoe::ledger_put(PMOE_LEDGER_JOIN, ce);
  return rc;
}

extern "C" int pmoe_copy_sync(pmoe_copy_engine* ce) {
  pmoe::clear_error();
  if (!ce) return pmoe::fail(PMOE_EINVAL, "copy_sync: null engine");
  int first_err = PMOE_OK;
  for (hipStream_t s : ce->streams) {
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess && first_err == PMOE_OK) first_err = pmoe::hip_fail(e, "copy_sync");
  }
  if (first_err == PMOE_OK) pmoe::ledger_put(PMOE_LEDGER_HOST_SYNC, ce);
  return first_err;
}

extern "C" int64_t pmoe_copy_bytes(pmoe_copy_engine* ce) { return ce ? ce->bytes : 0; }
