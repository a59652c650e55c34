// MoE layer orchestration: workspace layout, combine, and the public expert
// entry points (seam, experts+combine, whole block).
//
// Replaces StreamedSwitchGLU's compute (streaming.py:587-641, :768-841) and the
// parent block's combine `(y * scores[..., None]).sum(axis=-2)` plus the
// shared-expert add (restated tests/test_stream.py:198).  The combine is a
// fixed-order fp32 reduction: out[n] = fma over k = 0..K-1 of w[n,k]*y[n,k],
// then the shared expert, so results do not depend on scheduling.
#include <mutex>
#include <string>

#include "pmoe_internal.h"
#include "pmoe_kernels.h"
#include "route_common.h"

namespace pmoe {

int prefill_experts(const pmoe_geom* g, const uint8_t* slab, const uint16_t* x, int n, int kk,
                    const int32_t* order, const int4* tiles, const int32_t* n_tiles, int tile_m,
                    int max_tiles, uint16_t* h, void* y, int y_f32, hipStream_t st);
int prefill_tile_rows(int n, int kk, int n_experts);
int prefill_min_tile_rows();
bool prefill_wanted(const pmoe_geom* g, int n, int kk, int n_ids);

namespace {

constexpr size_t kAlign = 256;
constexpr size_t kSyncBytes = kDecodeSyncBytes;  // DecodeSync header at workspace offset 0

struct MoeWs {
  DecodeSync* sync = nullptr;     // first kSyncBytes of the workspace
  float* logits = nullptr;        // [n, E]
  float* shared_logit = nullptr;  // [n]
  int32_t* order = nullptr;       // [rows]
  int32_t* inv = nullptr;         // [rows]
  int32_t* counts = nullptr;      // [n_ids]
  int32_t* offsets = nullptr;     // [n_ids + 1]
  int32_t* active = nullptr;      // [n_ids]
  int32_t* n_active = nullptr;    // [1]
  int4* tiles = nullptr;          // [max_tiles] {slot, first row, rows, offset}
  int32_t* n_tiles = nullptr;     // [1]
  uint16_t* h = nullptr;          // [rows, inter] bf16
  float* y = nullptr;             // [rows, hidden] (bf16 or f32 per-slot outputs)
  void* dws = nullptr;            // dispatch scratch
  size_t dws_bytes = 0;
  void* record = nullptr;         // decode routing record
  int max_tiles = 0;
};

struct Carver {
  uint8_t* base;
  size_t off = 0;
  template <class T>
  T* take(size_t count) {
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += (count * sizeof(T) + kAlign - 1) / kAlign * kAlign;
    return p;
  }
};

size_t carve(const pmoe_geom* g, int n, int k, int shared, int n_experts, void* base,
             MoeWs* w) {
  const int kk = k + (shared ? 1 : 0);
  const size_t rows = size_t(n) * kk;
  const int n_ids = n_experts + (shared ? 1 : 0);
  Carver c{static_cast<uint8_t*>(base)};
  MoeWs t;
  t.sync = reinterpret_cast<DecodeSync*>(c.take<uint8_t>(kSyncBytes));
  t.logits = c.take<float>(size_t(n) * (n_experts + 1));
  t.shared_logit = c.take<float>(size_t(n));
  t.order = c.take<int32_t>(rows);
  t.inv = c.take<int32_t>(rows);
  t.counts = c.take<int32_t>(n_ids);
  t.offsets = c.take<int32_t>(n_ids + 1);
  t.active = c.take<int32_t>(n_ids);
  t.n_active = c.take<int32_t>(1);
  // tile capacity for the shortest prefill tiles
  t.max_tiles = int(rows / prefill_min_tile_rows()) + n_ids + 1;
  t.tiles = c.take<int4>(t.max_tiles);
  t.n_tiles = c.take<int32_t>(1);
  t.h = c.take<uint16_t>(rows * g->inter);
  t.y = c.take<float>(rows * g->hidden);
  t.dws_bytes = dispatch_workspace(int(rows), n_ids);
  t.dws = c.take<uint8_t>(t.dws_bytes);
  t.record = c.take<uint8_t>(decode_record_bytes());
  if (w) *w = t;
  return c.off;
}

// y: the per-slot expert outputs [n*kk, d] in bf16, as the reference's
// gather_qmm returns them; 8 outputs per thread.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y,
                                                      const float* __restrict__ w,
                                                      const int32_t* __restrict__ inv,
                                                      const float* __restrict__ shared_logit,
                                                      int has_shared, int k, int kk, int d,
                                                      uint16_t* __restrict__ out) {
  const int n = blockIdx.y;
  const int d0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (d0 >= d) return;
  float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < kk; ++c) {
    const size_t r = size_t(n) * kk + c;
    if (inv[r] < 0) continue;  // dropped id: contributes nothing
    float wt;
    if (c < k)
      wt = w[size_t(n) * k + c];
    else
      wt = shared_logit ? psigmoid(shared_logit[n]) : 1.0f;
    const uint4 v = *reinterpret_cast<const uint4*>(y + r * d + d0);
    const uint32_t p[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] = __builtin_fmaf(wt, bf16lo(p[i]), a[2 * i]);
      a[2 * i + 1] = __builtin_fmaf(wt, bf16hi(p[i]), a[2 * i + 1]);
    }
  }
  uint4 o;
  o.x = uint32_t(f2bf(a[0])) | (uint32_t(f2bf(a[1])) << 16);
  o.y = uint32_t(f2bf(a[2])) | (uint32_t(f2bf(a[3])) << 16);
  o.z = uint32_t(f2bf(a[4])) | (uint32_t(f2bf(a[5])) << 16);
  o.w = uint32_t(f2bf(a[6])) | (uint32_t(f2bf(a[7])) << 16);
  *reinterpret_cast<uint4*>(out + size_t(n) * d + d0) = o;
}

// Same reduction over bf16 per-slot outputs (the seam's [N, K, D]), for
// callers that ran the experts in several passes.
__global__ __launch_bounds__(256) void combine_bf16_kernel(const uint16_t* __restrict__ y,
                                                           const float* __restrict__ w,
                                                           const uint16_t* __restrict__ shared_y,
                                                           const float* __restrict__ shared_logit,
                                                           int k, int d,
                                                           uint16_t* __restrict__ out) {
  const int n = blockIdx.y;
  const int d0 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (d0 >= d) return;
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto add = [&](float wt, const uint16_t* src) {
    const uint2 v = *reinterpret_cast<const uint2*>(src + d0);
    a[0] = __builtin_fmaf(wt, bf16lo(v.x), a[0]);
    a[1] = __builtin_fmaf(wt, bf16hi(v.x), a[1]);
    a[2] = __builtin_fmaf(wt, bf16lo(v.y), a[2]);
    a[3] = __builtin_fmaf(wt, bf16hi(v.y), a[3]);
  };
  for (int c = 0; c < k; ++c) add(w[size_t(n) * k + c], y + (size_t(n) * k + c) * d);
  if (shared_y) add(shared_logit ? psigmoid(shared_logit[n]) : 1.0f, shared_y + size_t(n) * d);
  uint2 o;
  o.x = uint32_t(f2bf(a[0])) | (uint32_t(f2bf(a[1])) << 16);
  o.y = uint32_t(f2bf(a[2])) | (uint32_t(f2bf(a[3])) << 16);
  *reinterpret_cast<uint2*>(out + size_t(n) * d + d0) = o;
}

__global__ __launch_bounds__(256) void zero_dropped_rows_kernel(const int32_t* __restrict__ inv,
                                                                int rows, int d,
                                                                uint16_t* __restrict__ y) {
  const int r = blockIdx.y;
  if (r >= rows || inv[r] >= 0) return;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < d; i += gridDim.x * 256) y[size_t(r) * d + i] = 0;
}

int check_geom(const pmoe_geom* g) {
  PMOE_REQUIRE(g != nullptr, "null geometry");
  PMOE_REQUIRE(g->bits == 4 || g->bits == 6, "geometry: bits must be 4 or 6");
  PMOE_REQUIRE(g->group == 64, "geometry: group must be 64");
  PMOE_REQUIRE(g->hidden > 0 && g->hidden % 64 == 0 && g->inter > 0 && g->inter % 64 == 0,
               "geometry: hidden and inter must be multiples of 64");
  PMOE_REQUIRE(g->hidden <= 8192 && g->inter <= 8192, "geometry: dims above 8192");
  return PMOE_OK;
}

// The routing configuration, checked once before any path is chosen (the
// one-launch decode, the three-launch decode and the prefill routing kernels
// all assume it): a known scoring, 1 <= k <= min(16, E), and for sigmoid
// scoring groups that divide E, hold at least 2 experts, and keep enough
// experts for k.
int check_route_cfg(const pmoe_route_cfg* rc) {
  const int e = rc->n_experts, k = rc->top_k;
  PMOE_REQUIRE(rc->scoring == PMOE_SCORE_SOFTMAX || rc->scoring == PMOE_SCORE_SIGMOID,
               "routing: unknown scoring");
  PMOE_REQUIRE(k >= 1 && k <= kRouteMaxK && k <= e, "routing: top_k must be 1..min(16, E)");
  if (rc->scoring == PMOE_SCORE_SIGMOID) {
    const int g = rc->n_group, tg = rc->topk_group;
    PMOE_REQUIRE(g >= 1 && g <= 64 && e % g == 0, "routing: n_group must divide E and be <= 64");
    PMOE_REQUIRE(tg >= 1 && tg <= g, "routing: topk_group must be 1..n_group");
    PMOE_REQUIRE(g == 1 || e / g >= 2, "routing: groups need at least 2 experts");
    PMOE_REQUIRE(k <= (e / g) * tg, "routing: top_k exceeds the experts of the kept groups");
  }
  return PMOE_OK;
}

// Dispatch + the three projections (+ SwiGLU) for rows = n*kk flat rows.
// y receives [rows, hidden] (f32 when y_f32, else bf16).
int run_experts(const pmoe_geom* g, const uint8_t* slab, const int32_t* table, int n_experts,
                int shared_slot, const uint16_t* x, const int32_t* inds, int n, int k, int kk,
                int max_rows_per_expert, const MoeWs& w, void* y, int y_f32, hipStream_t st) {
  const int rows = n * kk;
  const int n_ids = n_experts + (kk > k ? 1 : 0);
  const bool prefill = prefill_wanted(g, n, kk, n_ids);
  const int tm = prefill ? prefill_tile_rows(n, kk, n_experts) : 0;
  // the tile list carries the slots of this table
  int rc = dispatch_ext(inds, rows, k, kk, n_ids, w.order, w.counts, w.offsets, w.inv, w.active,
                        w.n_active, tm, w.tiles, w.n_tiles, table, shared_slot, w.dws,
                        w.dws_bytes, st);
  if (rc) return rc;
  if (prefill)
    return prefill_experts(g, slab, x, n, kk, w.order, w.tiles, w.n_tiles, tm,
                           std::min(rows / tm + n_ids + 1, w.max_tiles), w.h, y, y_f32, st);
  const int max_experts = rows < n_ids ? rows : n_ids;
  GemvArgs a{};
  a.slab = slab;
  a.expert_bytes = g->expert_bytes;
  a.table = table;
  a.n_experts = n_experts;
  a.shared_slot = shared_slot;
  a.active = w.active;
  a.n_active = w.n_active;
  a.counts = w.counts;
  a.offsets = w.offsets;
  a.order = w.order;
  a.kk = kk;
  // gate + up -> h
  a.p0 = {g->off[PMOE_GATE_W], g->off[PMOE_GATE_S], g->off[PMOE_GATE_B]};
  a.p1 = {g->off[PMOE_UP_W], g->off[PMOE_UP_S], g->off[PMOE_UP_B]};
  a.rows_out = g->inter;
  a.cols = g->hidden;
  a.act = x;
  a.act_stride = g->hidden;
  a.act_by_token = 1;
  a.out = w.h;
  a.out_stride = g->inter;
  a.out_f32 = 0;
  rc = qgemv(a, g->bits, true, max_experts, max_rows_per_expert, st);
  if (rc) return rc;
  // down -> y
  a.p0 = {g->off[PMOE_DOWN_W], g->off[PMOE_DOWN_S], g->off[PMOE_DOWN_B]};
  a.p1 = a.p0;
  a.rows_out = g->hidden;
  a.cols = g->inter;
  a.act = w.h;
  a.act_stride = g->inter;
  a.act_by_token = 0;
  a.out = y;
  a.out_stride = g->hidden;
  a.out_f32 = y_f32;
  return qgemv(a, g->bits, false, max_experts, max_rows_per_expert, st);
}

// Decode path for n tokens: the one-launch layer for a single token (where
// it is the faster one), the three-launch decode for more.  The environment
// can pin either: PMOE_DECODE_FUSED=1 selects the one-launch layer for every
// decode batch it covers, 0 never (read per call, so the paths can be
// compared).
bool fused_enabled(int n) {
  const char* v = getenv("PMOE_DECODE_FUSED");
  if (v && v[0] == '1') return true;
  if (v && v[0] == '0') return false;
  return n == 1;
}

// Decode block path: the fused one-launch layer (decode_fused.hip) when it
// covers the shape, else the router launch (logits + shared gate column;
// with several tokens its last block also routes and publishes the record),
// then gate/up and down+combine (one token: each block recomputes the
// routing in its prologue).
int decode_block(const pmoe_geom* g, const pmoe_route_cfg* rc, const uint8_t* slab,
                 const int32_t* table, const uint16_t* gate_w, const float* score_bias,
                 const float* logit_bias, const uint16_t* x, int n, int shared_slot,
                 const uint16_t* shared_gate, uint16_t* out, int32_t* inds_out, float* w_out,
                 const MoeWs& w, hipStream_t st) {
  const int e = rc->n_experts, k = rc->top_k;
  const int shared = shared_slot >= 0 ? 1 : 0;
  const int kk = k + shared;
  const uint16_t* extra = (shared && shared_gate) ? shared_gate : nullptr;
  RouteDev rt{};
  rt.logits = w.logits;
  rt.ld = e + (extra ? 1 : 0);
  rt.bias = score_bias;
  rt.scoring = rc->scoring;
  rt.n = n;
  rt.e = e;
  rt.k = k;
  rt.kk = kk;
  rt.norm = rc->norm_topk_prob;
  rt.n_group = rc->n_group;
  rt.topk_group = rc->topk_group;
  rt.scale = rc->routed_scale;
  rt.shared_gate = extra ? 1 : 0;
  GemvArgs gu{};
  gu.slab = slab;
  gu.expert_bytes = g->expert_bytes;
  gu.table = table;
  gu.n_experts = e;
  gu.shared_slot = shared_slot;
  gu.kk = kk;
  gu.p0 = {g->off[PMOE_GATE_W], g->off[PMOE_GATE_S], g->off[PMOE_GATE_B]};
  gu.p1 = {g->off[PMOE_UP_W], g->off[PMOE_UP_S], g->off[PMOE_UP_B]};
  gu.rows_out = g->inter;
  gu.cols = g->hidden;
  gu.act = x;
  gu.act_stride = g->hidden;
  gu.act_by_token = 1;
  gu.out = w.h;
  gu.out_stride = g->inter;
  GemvArgs dn = gu;
  dn.p0 = {g->off[PMOE_DOWN_W], g->off[PMOE_DOWN_S], g->off[PMOE_DOWN_B]};
  dn.p1 = dn.p0;
  dn.rows_out = g->hidden;
  dn.cols = g->inter;
  dn.act = w.h;
  dn.act_stride = g->inter;
  dn.act_by_token = 0;
  dn.out = nullptr;
  const RouterIn ri{x, gate_w, extra, logit_bias, g->hidden, w.logits,
                    reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(w.sync) +
                                                kRouteArriveOffset)};
  if (fused_enabled(n)) {
    // one token with 8 picks that the expert-per-XCD layer does not route
    // (sigmoid or grouped scoring, a shared expert): the router launch,
    // then the given-ids expert-per-XCD launch on its picks, combining fp32
    // columns as the expert-split down does
    if (n == 1 && k == kXcdCount && !extra &&
        !decode_xcd_covers(gu, dn, rt, g->bits, false) &&
        experts_xcd_covers(gu, dn, g->bits, shared_slot)) {
      const int r1 = decode_route(gu, rt, inds_out, w_out, w.record, ri, st);
      if (r1) return r1;
      const int r3 = experts_xcd(gu, dn, g->bits, e, inds_out, w_out, shared_slot, out, w.sync,
                                 st, false);
      if (r3 != kDecodeFusedDeclined) return r3;
      return fail(PMOE_ESTATE, "decode: the given-ids launch declined a shape it covers");
    }
    const int r2 = decode_fused(gu, dn, rt, g->bits, x, gate_w, extra, logit_bias, inds_out, w_out,
                                out, w.sync, st);
    if (r2 != kDecodeFusedDeclined) return r2;
  }
  dn.out = w.y;  // fp32 per-slot outputs when the down runs expert-split
  return decode_routed(gu, dn, rt, g->bits, inds_out, w_out, out, w.record, ri, st);
}

int experts_and_combine(const pmoe_geom* g, const uint8_t* slab, const int32_t* table,
                        int n_experts, const uint16_t* x, const int32_t* inds, const float* wts,
                        int n, int k, int shared_slot, const uint16_t* shared_gate, int max_rpe,
                        uint16_t* out, const MoeWs& w, hipStream_t st) {
  const int shared = shared_slot >= 0 ? 1 : 0;
  const int kk = k + shared;
  if (n == 1 && k == kXcdCount && !(shared && shared_gate)) {
    // one token, eight columns: the expert-per-XCD launch (same outputs)
    GemvArgs gu{};
    gu.slab = slab;
    gu.expert_bytes = g->expert_bytes;
    gu.table = table;
    gu.n_experts = n_experts;
    gu.shared_slot = shared_slot;
    gu.kk = kk;
    gu.p0 = {g->off[PMOE_GATE_W], g->off[PMOE_GATE_S], g->off[PMOE_GATE_B]};
    gu.p1 = {g->off[PMOE_UP_W], g->off[PMOE_UP_S], g->off[PMOE_UP_B]};
    gu.rows_out = g->inter;
    gu.cols = g->hidden;
    gu.act = x;
    gu.act_stride = g->hidden;
    gu.act_by_token = 1;
    GemvArgs dn = gu;
    dn.p0 = {g->off[PMOE_DOWN_W], g->off[PMOE_DOWN_S], g->off[PMOE_DOWN_B]};
    dn.p1 = dn.p0;
    dn.rows_out = g->hidden;
    dn.cols = g->inter;
    const int r = experts_xcd(gu, dn, g->bits, n_experts, inds, wts, shared_slot, out, w.sync, st);
    if (r != kDecodeFusedDeclined) return r;
  }
  int rc = run_experts(g, slab, table, n_experts, shared_slot, x, inds, n, k, kk, max_rpe, w,
                       w.y, 0, st);
  if (rc) return rc;
  const float* sl = nullptr;
  if (shared && shared_gate) {
    rc = router_logits(x, shared_gate, nullptr, n, g->hidden, 1, w.shared_logit, st);
    if (rc) return rc;
    sl = w.shared_logit;
  }
  dim3 grid((g->hidden / 8 + 255) / 256, n);
  ProfScope prof_scope(K_COMBINE, st);
  combine_kernel<<<grid, 256, 0, st>>>(reinterpret_cast<const uint16_t*>(w.y), wts, w.inv, sl,
                                       shared, k, kk, g->hidden, out);
  PMOE_LAUNCH_CHECK("combine_kernel");
  return PMOE_OK;
}

}  // namespace

}  // namespace pmoe

using pmoe::MoeWs;

extern "C" size_t pmoe_moe_workspace(const pmoe_geom* g, int n, int k, int shared,
                                     int n_experts) {
  if (!g || n < 0 || k <= 0 || n_experts <= 0) return 0;
  return pmoe::carve(g, n, k, shared, n_experts, nullptr, nullptr);
}

__global__ void workspace_init_kernel(uint32_t* p, int words) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x)
    p[i] = 0;
}

extern "C" int pmoe_moe_workspace_init(void* ws, size_t ws_bytes, void* stream) {
  pmoe::clear_error();
  PMOE_REQUIRE(ws != nullptr, "moe_workspace_init: null workspace");
  PMOE_REQUIRE(ws_bytes >= pmoe::kSyncBytes, "moe_workspace_init: workspace too small");
  workspace_init_kernel<<<64, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<uint32_t*>(ws), int(pmoe::kSyncBytes / 4));
  PMOE_LAUNCH_CHECK("workspace_init_kernel");
  return PMOE_OK;
}

extern "C" int pmoe_moe_workspace_status(const void* ws, uint32_t* error, void* stream) {
  pmoe::clear_error();
  PMOE_REQUIRE(ws != nullptr && error != nullptr, "moe_workspace_status: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const pmoe::DecodeSync* sy = static_cast<const pmoe::DecodeSync*>(ws);
  PMOE_HIP(hipMemcpyAsync(error, &sy->error, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  PMOE_HIP(hipStreamSynchronize(st));
  return PMOE_OK;
}

extern "C" int pmoe_moe_workspace_error_async(const void* ws, uint32_t* host_dst,
                                              void* stream) {
  pmoe::clear_error();
  PMOE_REQUIRE(ws != nullptr && host_dst != nullptr, "moe_workspace_error_async: null pointer");
  const pmoe::DecodeSync* sy = static_cast<const pmoe::DecodeSync*>(ws);
  PMOE_HIP(hipMemcpyAsync(host_dst, &sy->error, sizeof(uint32_t), hipMemcpyDeviceToHost,
                          static_cast<hipStream_t>(stream)));
  return PMOE_OK;
}

extern "C" int pmoe_switch_glu(const pmoe_geom* g, const void* slab, const int32_t* table,
                               int n_experts, const void* x, const int32_t* inds, int n, int k,
                               void* y, void* ws, size_t ws_bytes, void* stream) {
  pmoe::clear_error();
  int rc = pmoe::check_geom(g);
  if (rc) return rc;
  PMOE_REQUIRE(slab && table && x && inds && y, "switch_glu: null pointer");
  PMOE_REQUIRE(n >= 0 && k > 0 && n_experts > 0 && n_experts <= 1023, "switch_glu: bad shape");
  if (n == 0) return PMOE_OK;
  const size_t need = pmoe::carve(g, n, k, 0, n_experts, nullptr, nullptr);
  if (!ws || ws_bytes < need) return pmoe::fail(PMOE_ESPACE, "switch_glu: workspace too small");
  MoeWs w;
  pmoe::carve(g, n, k, 0, n_experts, ws, &w);
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = pmoe::run_experts(g, static_cast<const uint8_t*>(slab), table, n_experts, -1,
                         static_cast<const uint16_t*>(x), inds, n, k, k, n * k, w, y, 0, st);
  if (rc) return rc;
  dim3 grid(1, n * k);
  pmoe::zero_dropped_rows_kernel<<<grid, 256, 0, st>>>(w.inv, n * k, g->hidden,
                                                       static_cast<uint16_t*>(y));
  PMOE_LAUNCH_CHECK("zero_dropped_rows_kernel");
  return PMOE_OK;
}

extern "C" int pmoe_moe_experts(const pmoe_geom* g, const void* slab, const int32_t* table,
                                int n_experts, const void* x, const int32_t* inds,
                                const float* weights, int n, int k, int shared_slot,
                                const void* shared_gate, void* out, void* ws, size_t ws_bytes,
                                void* stream) {
  pmoe::clear_error();
  int rc = pmoe::check_geom(g);
  if (rc) return rc;
  PMOE_REQUIRE(slab && table && x && inds && weights && out, "moe_experts: null pointer");
  PMOE_REQUIRE(n >= 0 && k > 0 && n_experts > 0 && n_experts <= 1023, "moe_experts: bad shape");
  if (n == 0) return PMOE_OK;
  const int shared = shared_slot >= 0 ? 1 : 0;
  const size_t need = pmoe::carve(g, n, k, shared, n_experts, nullptr, nullptr);
  if (!ws || ws_bytes < need) return pmoe::fail(PMOE_ESPACE, "moe_experts: workspace too small");
  MoeWs w;
  pmoe::carve(g, n, k, shared, n_experts, ws, &w);
  return pmoe::experts_and_combine(
      g, static_cast<const uint8_t*>(slab), table, n_experts, static_cast<const uint16_t*>(x),
      inds, weights, n, k, shared_slot, static_cast<const uint16_t*>(shared_gate), n * (k + 1),
      static_cast<uint16_t*>(out), w, static_cast<hipStream_t>(stream));
}

extern "C" int pmoe_moe_block(const pmoe_geom* g, const pmoe_route_cfg* rc_cfg, const void* slab,
                              const int32_t* table, const void* gate_w, const float* score_bias,
                              const float* logit_bias, const void* x, int n, int shared_slot,
                              const void* shared_gate, void* out, int32_t* inds_out,
                              float* weights_out, void* ws, size_t ws_bytes, void* stream) {
  pmoe::clear_error();
  int rc = pmoe::check_geom(g);
  if (rc) return rc;
  PMOE_REQUIRE(rc_cfg != nullptr, "moe_block: null routing config");
  PMOE_REQUIRE(slab && table && gate_w && x && out && inds_out && weights_out,
               "moe_block: null pointer");
  const int e = rc_cfg->n_experts, k = rc_cfg->top_k;
  PMOE_REQUIRE(n >= 0 && k > 0 && e > 0 && e <= 1023, "moe_block: bad shape");
  rc = pmoe::check_route_cfg(rc_cfg);
  if (rc) return rc;
  if (n == 0) return PMOE_OK;
  const int shared = shared_slot >= 0 ? 1 : 0;
  const size_t need = pmoe::carve(g, n, k, shared, e, nullptr, nullptr);
  if (!ws || ws_bytes < need) return pmoe::fail(PMOE_ESPACE, "moe_block: workspace too small");
  MoeWs w;
  pmoe::carve(g, n, k, shared, e, ws, &w);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const int kk = k + shared;
  const bool decode = n * kk <= pmoe::kRouteMaxRows && e + 1 <= pmoe::kRouteMaxIds &&
                      k <= pmoe::kRouteMaxK && !pmoe::prefill_wanted(g, n, kk, e + shared) &&
                      (rc_cfg->scoring == PMOE_SCORE_SOFTMAX ||
                       (e <= pmoe::kRouteMaxSigE && rc_cfg->topk_group <= 8));
  if (decode) {
    if (rc_cfg->scoring == PMOE_SCORE_SIGMOID)
      PMOE_REQUIRE(score_bias != nullptr, "moe_block: sigmoid scoring needs score_bias");
    return pmoe::decode_block(g, rc_cfg, static_cast<const uint8_t*>(slab), table,
                              static_cast<const uint16_t*>(gate_w), score_bias, logit_bias, xb, n,
                              shared_slot, static_cast<const uint16_t*>(shared_gate),
                              static_cast<uint16_t*>(out), inds_out, weights_out, w, st);
  }
  rc = pmoe::router_logits(xb, static_cast<const uint16_t*>(gate_w), logit_bias, n, g->hidden, e,
                           w.logits, st);
  if (rc) return rc;
  if (rc_cfg->scoring == PMOE_SCORE_SOFTMAX) {
    rc = pmoe::route_softmax(w.logits, n, e, k, rc_cfg->norm_topk_prob, inds_out, weights_out, st);
  } else if (rc_cfg->scoring == PMOE_SCORE_SIGMOID) {
    PMOE_REQUIRE(score_bias != nullptr, "moe_block: sigmoid scoring needs score_bias");
    rc = pmoe::route_sigmoid(w.logits, score_bias, n, e, rc_cfg->n_group, rc_cfg->topk_group, k,
                             rc_cfg->norm_topk_prob, rc_cfg->routed_scale, inds_out, weights_out,
                             st);
  } else {
    return pmoe::fail(PMOE_EINVAL, "moe_block: unknown scoring");
  }
  if (rc) return rc;
  return pmoe::experts_and_combine(g, static_cast<const uint8_t*>(slab), table, e, xb, inds_out,
                                   weights_out, n, k, shared_slot,
                                   static_cast<const uint16_t*>(shared_gate), n,
                                   static_cast<uint16_t*>(out), w, st);
}

// ---------------------------------------------------------------- no allocation
//
// pmoe_moe_block for callers that cannot allocate (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc): the
// workspace is carved from `scratch`, a file-scope device array of
// kStaticScratchBytes that each GPU holds until the process ends.  In host
// code `scratch` only names the symbol: its device address is looked up with
// hipGetSymbolAddress once per device (with that device current) and kept in
// g_scratch_ptr[device]; only that address is ever passed to kernels.  The
// same first call zeroes the array's synchronisation header with a kernel
// (so it must not be made under graph capture: it returns PMOE_ESTATE);
// every later call leaves the header consistent, as pmoe_moe_block does for
// a caller's workspace.  All calls on one GPU share the array, so calls that
// overlap on one GPU (two streams, two threads) race.

namespace {

constexpr size_t kStaticScratchBytes = size_t(32) << 20;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

}  // namespace

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

static int scratch_for_device(void** out, hipStream_t st) {
  int dev = -1;
  PMOE_HIP(hipGetDevice(&dev));
  PMOE_REQUIRE(dev >= 0 && dev < kMaxDevices, "moe_block_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // the header's zeroing must run once, eagerly: captured into a graph it
    // would run again at every replay and wipe the counters the calls keep
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    PMOE_HIP(hipStreamIsCapturing(st, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return pmoe::fail(PMOE_ESTATE,
                        "moe_block_noalloc: the first call on a device sets up its static "
                        "scratch and must run outside graph capture");
    void* p = nullptr;
    PMOE_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    workspace_init_kernel<<<64, 256, 0, st>>>(static_cast<uint32_t*>(p),
                                              int(pmoe::kSyncBytes / 4));
    PMOE_LAUNCH_CHECK("workspace_init_kernel (static scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PMOE_OK;
}

extern "C" int pmoe_moe_block_noalloc(const pmoe_geom* g, const pmoe_route_cfg* rc_cfg,
                                      const void* slab, const int32_t* table, const void* gate_w,
                                      const float* score_bias, const float* logit_bias,
                                      const void* x, int n, int shared_slot,
                                      const void* shared_gate, void* out, int32_t* inds_out,
                                      float* weights_out, void* stream) {
  pmoe::clear_error();
  int rc = pmoe::check_geom(g);
  if (rc) return rc;
  PMOE_REQUIRE(rc_cfg != nullptr, "moe_block_noalloc: null routing config");
  PMOE_REQUIRE(n >= 0 && rc_cfg->top_k > 0 && rc_cfg->n_experts > 0 &&
                   rc_cfg->n_experts <= 1023,
               "moe_block_noalloc: bad shape");
  const size_t need = pmoe::carve(g, n, rc_cfg->top_k, shared_slot >= 0 ? 1 : 0,
                                  rc_cfg->n_experts, nullptr, nullptr);
  if (need > kStaticScratchBytes)
    return pmoe::fail(PMOE_ESPACE, "moe_block_noalloc: this call needs " + std::to_string(need) +
                                       " bytes of scratch; the static scratch holds " +
                                       std::to_string(kStaticScratchBytes) +
                                       " (decode-sized batches); use pmoe_moe_block with a "
                                       "caller workspace");
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  rc = scratch_for_device(&ws, st);
  if (rc) return rc;
  return pmoe_moe_block(g, rc_cfg, slab, table, gate_w, score_bias, logit_bias, x, n, shared_slot,
                        shared_gate, out, inds_out, weights_out, ws, kStaticScratchBytes, stream);
}

namespace pmoe {
namespace {

// One block: each thread counts its strided ids, a wave sum, then one
// atomic per wave (vector atomics only).
__global__ __launch_bounds__(256) void count_missing_kernel(const int32_t* __restrict__ table,
                                                            const int32_t* __restrict__ ids,
                                                            int n, int n_experts,
                                                            int32_t* __restrict__ counter) {
  int c = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int e = ids[i];
    c += (e >= 0 && e < n_experts && table[e] < 0) ? 1 : 0;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
  if ((threadIdx.x & 63) == 0 && c) atomicAdd(counter, c);
}

}  // namespace
}  // namespace pmoe

extern "C" int pmoe_count_missing(const int32_t* table, const int32_t* ids, int n, int n_experts,
                                  int32_t* counter, void* stream) {
  pmoe::clear_error();
  PMOE_REQUIRE(table && counter && (n == 0 || ids), "count_missing: null pointer");
  PMOE_REQUIRE(n >= 0 && n_experts > 0, "count_missing: bad shape");
  if (n == 0) return PMOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  pmoe::count_missing_kernel<<<1, 256, 0, st>>>(table, ids, n, n_experts, counter);
  PMOE_LAUNCH_CHECK("count_missing_kernel");
  return PMOE_OK;
}

extern "C" int pmoe_combine(const void* y, const float* weights, int n, int k, int hidden,
                            const void* shared_y, const float* shared_logit, void* out,
                            void* stream) {
  pmoe::clear_error();
  PMOE_REQUIRE(y && weights && out, "combine: null pointer");
  PMOE_REQUIRE(n >= 0 && n <= 65535 && k > 0 && hidden > 0 && hidden % 4 == 0,
               "combine: bad shape");
  PMOE_REQUIRE(!shared_logit || shared_y, "combine: shared_logit without shared_y");
  PMOE_REQUIRE((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out) |
                reinterpret_cast<uintptr_t>(shared_y)) % 8 == 0,
               "combine: y/out/shared_y must be 8-byte aligned");
  if (n == 0) return PMOE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid((hidden / 4 + 255) / 256, n);
  pmoe::ProfScope prof_scope(pmoe::K_COMBINE, st);
  pmoe::combine_bf16_kernel<<<grid, 256, 0, st>>>(
      static_cast<const uint16_t*>(y), weights, static_cast<const uint16_t*>(shared_y),
      shared_logit, k, hidden, static_cast<uint16_t*>(out));
  PMOE_LAUNCH_CHECK("combine_bf16_kernel");
  return PMOE_OK;
}
