// Grouped dequant-GEMV for decode-sized batches (few rows per expert).
//
// Replaces the three mx.gather_qmm calls of the slab path (_run_slab ->
// _slab_rows -> _gather_proj, streaming.py:587-641 and :504-536) and the
// SwiGLU between them (streaming.py:640).  One launch computes a projection
// for every active expert at once: blockIdx.y picks the expert (ascending id,
// from the dispatch), blockIdx.x a tile of output rows, and each wave walks its
// rows, each lane owning units of the row (16-byte chunks for 4-bit, whole
// 64-value quant groups for 6-bit; gemv_common.h).
//
// The per-lane arithmetic (128-bit packed loads, in-register (128+q) bf16
// pairs, v_dot2_f32_bf16, xor-butterfly row sums) is in gemv_common.h.  The
// gate/up launch (DUAL) computes both projections of a row together and
// writes h = silu(g)*u as bf16.
#include <type_traits>

#include "gemv_common.h"
#include "pmoe_internal.h"
#include "pmoe_kernels.h"
#include "route_common.h"
#include "router_tile.h"

namespace pmoe {

namespace {

// Zero outputs of an expert whose table entry is -1 (not resident): it
// contributes exact zero rows (streaming.py:715-719).
__device__ __forceinline__ void store_zero_rows(const GemvArgs& a, int m_total,
                                                const int32_t* rlist, int row0, int rows) {
  for (int m = 0; m < m_total; ++m) {
    const int r = rlist[m];
    for (int i = threadIdx.x; i < rows; i += 256) {
      const int o = row0 + i;
      if (o >= a.rows_out) break;
      if (a.out_f32)
        static_cast<float*>(a.out)[size_t(r) * a.out_stride + o] = 0.0f;
      else
        static_cast<uint16_t*>(a.out)[size_t(r) * a.out_stride + o] = 0;
    }
  }
}

// ---------------------------------------------------------------- kernels

// Expert-major grouped projection: blockIdx.y = active expert (from a
// dispatch in global memory), blockIdx.x = tile of 4*R*RPW output rows.
template <int UB, int LPR, int GPL, int R, bool DUAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PMOE_MIN_WAVES, 8))) void qgemv_kernel(
    const GemvArgs a) {
  constexpr int RPW = 64 / LPR;
  const int u = blockIdx.y;
  if (u >= *a.n_active) return;
  const int e = a.active[u];
  const int slot = e < a.n_experts ? a.table[e] : a.shared_slot;
  const int m_total = a.counts[e];
  const int32_t* rlist = a.order + a.offsets[e];
  const int row0 = blockIdx.x * (4 * R * RPW);
  if (slot < 0) {
    store_zero_rows(a, m_total, rlist, row0, 4 * R * RPW);
    return;
  }
  const int wrow0 = row0 + (threadIdx.x >> 6) * (R * RPW);
  auto act_row = [&](int r) {
    return a.act + size_t(a.act_by_token ? r / a.kk : r) * a.act_stride;
  };
  auto store = [&](int r, int, int o, float v) {
    const size_t idx = size_t(r) * a.out_stride + o;
    if (a.out_f32)
      static_cast<float*>(a.out)[idx] = v;
    else
      static_cast<uint16_t*>(a.out)[idx] = f2bf(v);
  };
  gemv_expert<UB, LPR, GPL, R, DUAL>(a, slot, m_total, rlist, wrow0, act_row, store);
}

// Decode gate/up with the routing computed in the block's prologue (see
// route_common.h): blockIdx.y = u-th active expert in ascending id order.
// Block (0, 0) also publishes the routing (inds_out, w_out).
// PRE: the routing record was written by the router launch (several
// tokens; router_route_kernel) and wave 0 gathers the expert's rows from it
// for the block; otherwise every block routes its one token itself and block
// (0, 0) publishes the record.  (Every wave gathering its own list, as the
// expert-split down does, made the Qwen3-235B-shaped batch-8 gate/up slower,
// 74.8 -> 78.3 us in rocprof.)
// More than 8 logits per lane (over 512 experts): the routing prologue's
// per-lane logit, key and payload arrays need more registers than the GEMV's
// occupancy floor leaves, so those variants run with two waves per SIMD.
template <int EPL>
constexpr int routed_min_waves() {
  return EPL > 8 ? 2 : PMOE_MIN_WAVES;
}

template <int UB, int LPR, int GPL, int R, int EPL, bool PRE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(routed_min_waves<EPL>(), 8))) void
gateup_routed_kernel(const GemvArgs a, const RouteDev rt, int32_t* inds_out, float* w_out,
                     RouteRecord* rec) {
  constexpr int RPW = 64 / LPR;
  __shared__ RouteLds L;
  __shared__ WaveTmp W[PRE ? 1 : 4];
  __shared__ int32_t s_rows[kRouteMaxRows];
  __shared__ int s_m;
  const int u = blockIdx.y;
  int slot;
  if (PRE) {
    const RouteOne one = load_route_one(rec, u);
    if (u >= one.n_active) return;
    slot = one.slot;
    if (threadIdx.x < 64) {
      const int m = wave_rows_of_record(rec, rt.n * rt.kk, one.e, s_rows);
      if (threadIdx.x == 0) s_m = m;
    }
  } else {
    const bool publish = blockIdx.x == 0 && blockIdx.y == 0;
    route_block<EPL, 4>(rt, L, W, publish ? inds_out : nullptr, w_out);
    if (publish)
      publish_route(L, rt.n * rt.kk, rec, a.table, a.n_experts, a.shared_slot);
    if (u >= L.n_active) return;
    const int e = L.active[u];
    slot = e < a.n_experts ? a.table[e] : a.shared_slot;
    if (threadIdx.x < 64) {
      const int m = wave_rows_of(L, rt.n * rt.kk, e, s_rows);
      if (threadIdx.x == 0) s_m = m;
    }
  }
  __syncthreads();
  const int row0 = blockIdx.x * (4 * R * RPW);
  if (slot < 0) {
    store_zero_rows(a, s_m, s_rows, row0, 4 * R * RPW);
    return;
  }
  const int wrow0 = row0 + (threadIdx.x >> 6) * (R * RPW);
  auto act_row = [&](int r) { return a.act + size_t(r / rt.kk) * a.act_stride; };
  auto store = [&](int r, int, int o, float v) {
    static_cast<uint16_t*>(a.out)[size_t(r) * a.out_stride + o] = f2bf(v);
  };
  gemv_expert<UB, LPR, GPL, R, true>(a, slot, s_m, s_rows, wrow0, act_row, store);
}

// Router launch of a decode call of several tokens whose last block also
// routes: every block stores its logits at device scope and then arrives at
// a counter; the block that arrives last (every logit visible) routes the
// tokens with its 8 waves (one token per wave per round; route_block, logits
// read at device scope), publishes the routing record (shared expert first)
// and the routing outputs, and resets the counter for the next launch.  No
// block waits for another, and the per-expert launches after it find the
// record ready.  Every block copies the slot table into LDS while its logits
// load, so the last one's record needs no further dependent read.
constexpr int kTailWaves = 8;

#ifdef PMOE_FUSED_TRACE
// Debug builds: realtime stamps of the router launch's phases, per block.
__device__ uint64_t g_rtrace[1024 * 8];
#define PMOE_RT_MARK(i)                                                              \
  do {                                                                               \
    if (threadIdx.x == 0)                                                            \
      g_rtrace[(blockIdx.y * gridDim.x + blockIdx.x) * 8 + (i)] =                   \
          __builtin_amdgcn_s_memrealtime();                                          \
  } while (0)
#else
#define PMOE_RT_MARK(i)
#endif

struct RouteTail {
  RouteDev rt;
  RouteRecord* rec;
  const int32_t* table;
  int n_experts, shared_slot;
  int32_t* inds_out;
  float* w_out;
  uint32_t* arrive;  // zero between launches
};

template <int TE, int TN, int UNR, bool FULL, int EPL>
__global__ __launch_bounds__(64 * kTailWaves) void router_route_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ w_extra, const float* __restrict__ bias, int n, int d, int e,
    int n_w, float* __restrict__ out, const RouteTail t) {
  __shared__ RouteLds L;
  __shared__ WaveTmp W[kTailWaves];
  __shared__ int32_t s_table[kRouteMaxIds];
  __shared__ int s_last;
  PMOE_RT_MARK(0);
  for (int i = threadIdx.x; i < t.n_experts; i += 64 * kTailWaves) s_table[i] = t.table[i];
  const int e0 = (blockIdx.x * kTailWaves + int(threadIdx.x >> 6)) * TE;
  if (e0 < e)
    router_tile<TE, TN, UNR, FULL, true>(x, w, w_extra, bias, n, d, e, n_w, out, e0,
                                         blockIdx.y * TN);
  PMOE_RT_MARK(1);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's logits have reached device scope
  __syncthreads();
  PMOE_RT_MARK(2);
  if (threadIdx.x == 0) {
    const uint32_t total = gridDim.x * gridDim.y;
    s_last = __hip_atomic_fetch_add(t.arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             total - 1;
  }
  __syncthreads();
  PMOE_RT_MARK(3);
  if (!s_last) return;
  if (threadIdx.x == 0) __hip_atomic_store(t.arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  route_block<EPL, kTailWaves, true>(t.rt, L, W, t.inds_out, t.w_out);
  PMOE_RT_MARK(4);
  publish_route(L, t.rt.n * t.rt.kk, t.rec, s_table, t.n_experts, t.shared_slot);
  PMOE_RT_MARK(5);
}

// Decode down projection + weighted combine, routing recomputed in the
// prologue.  Tile-major: block b owns output rows [b*T, b*T + T) for every
// active expert (wave w takes experts w, w+4, ...); each (flat row, output)
// value lands in LDS and the block then forms
//   out[n, o] = sum_c w[n, c] * y[n*kk + c, o],  c = 0..kk-1 in that order
// (shared expert last) -- no y buffer, no extra launch, no cross-block sync.
template <int UB, int LPR, int GPL, int R, int EPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PMOE_MIN_WAVES, 8))) void
down_routed_kernel(const GemvArgs a, const RouteDev rt, uint16_t* out, const RouteRecord* rec) {
  constexpr int RPW = 64 / LPR;
  constexpr int T = R * RPW;
  __shared__ RouteLds L;
  __shared__ int32_t s_rows[4][kRouteMaxRows];
  extern __shared__ float s_y[];  // [rows][T]
  const int wave = threadIdx.x >> 6;
  load_route(rec, rt.n * rt.kk, rt.e + (rt.kk > rt.k ? 1 : 0), L);
  const int rows = rt.n * rt.kk;
  const int row0 = blockIdx.x * T;
  for (int u = wave; u < L.n_active; u += 4) {
    const int e = L.active[u];
    const int m_total = wave_rows_of(L, rows, e, s_rows[wave]);
    const int slot = e < a.n_experts ? a.table[e] : a.shared_slot;
    if (slot < 0) {
      for (int m = 0; m < m_total; ++m)
        for (int t = threadIdx.x & 63; t < T; t += 64) s_y[s_rows[wave][m] * T + t] = 0.0f;
      continue;
    }
    auto act_row = [&](int r) { return a.act + size_t(r) * a.act_stride; };
    auto store = [&](int r, int st, int o, float v) { s_y[r * T + (o - row0)] = v; };
    gemv_expert<UB, LPR, GPL, R, false>(a, slot, m_total, s_rows[wave], row0, act_row, store);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < rt.n * T; i += 256) {
    const int n = i / T, t = i - n * T;
    const int o = row0 + t;
    if (o >= a.rows_out) continue;
    float acc = 0.0f;
    for (int col = 0; col < rt.kk; ++col)
      acc = __builtin_fmaf(L.w[n * rt.kk + col], s_y[(n * rt.kk + col) * T + t], acc);
    out[size_t(n) * a.rows_out + o] = f2bf(acc);
  }
}

// Decode down projection, expert-split (many active experts): blockIdx.y =
// u-th active expert of the routing record, blockIdx.x = tile of 4*R*RPW
// output rows; the expert's rows go to y[r, o] (fp32), combined afterwards
// by combine_y_kernel.  The tile-major down_routed_kernel gives each wave
// every fourth active expert, a serial chain that is latency-bound once
// dozens of experts are active; here every (expert, tile) is its own block.
// Per-row arithmetic and combine order are those of down_routed_kernel, so
// the results are bit-identical.
template <int UB, int LPR, int GPL, int R, int EPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PMOE_MIN_WAVES, 8))) void
down_split_kernel(const GemvArgs a, const RouteDev rt, float* y, const RouteRecord* rec) {
  constexpr int RPW = 64 / LPR;
  __shared__ int32_t s_rows[4][kRouteMaxRows];  // each wave's own list (the same rows)
  const int wave = threadIdx.x >> 6;
  const int u = blockIdx.y;
  const RouteOne one = load_route_one(rec, u);
  // rows first: their loads need not wait for the active count
  const int m = wave_rows_of_record(rec, rt.n * rt.kk, one.e, s_rows[wave]);
  if (u >= one.n_active) return;
  const int slot = one.slot;
  const int row0 = blockIdx.x * (4 * R * RPW);
  if (slot < 0) {  // exact zero rows (streaming.py:715-719)
    for (int i = threadIdx.x; i < m * 4 * R * RPW; i += 256) {
      const int o = row0 + i % (4 * R * RPW);
      if (o < a.rows_out) y[size_t(s_rows[wave][i / (4 * R * RPW)]) * a.rows_out + o] = 0.0f;
    }
    return;
  }
  const int wrow0 = row0 + wave * (R * RPW);
  auto act_row = [&](int r) { return a.act + size_t(r) * a.act_stride; };
  auto store = [&](int r, int, int o, float v) { y[size_t(r) * a.rows_out + o] = v; };
  gemv_expert<UB, LPR, GPL, R, false>(a, slot, m, s_rows[wave], wrow0, act_row, store);
}

// out[n, o] = sum_c w[n, c] * y[n*kk + c, o] in c order (fma chain from 0,
// as down_routed_kernel's combine).
__global__ __launch_bounds__(256) void combine_y_kernel(const float* __restrict__ y,
                                                        const RouteRecord* __restrict__ rec,
                                                        int kk, int d, uint16_t* __restrict__ out) {
  const int n = blockIdx.y;
  const int o = blockIdx.x * 256 + threadIdx.x;
  if (o >= d) return;
  float acc = 0.0f;
  for (int c = 0; c < kk; ++c)
    acc = __builtin_fmaf(rec->w[n * kk + c], y[size_t(n * kk + c) * d + o], acc);
  out[size_t(n) * d + o] = f2bf(acc);
}

// Row steps per wave: as many as fit next to the activations in a
// 3-waves-per-SIMD register budget (~150 VGPRs: GPL units of activation
// pairs, ~30 for addresses and sums, ~8 per unit of unpacked pairs in flight
// once a lane has 3 or more units, the rest for packed weights), at most 4.
template <int UB, int GPL, bool DUAL>
constexpr int rows_r() {
  constexpr int per_step = GPL * (Unit<UB>::kWords + 2) * (DUAL ? 2 : 1);
  constexpr int budget =
      150 - 30 - GPL * (Unit<UB>::kVals / 2 + 1) - (GPL >= 3 ? 8 * GPL : 0);
  constexpr int r = budget / per_step;
  if (PMOE_FORCE_R > 0) return PMOE_FORCE_R;
  // 6-bit (48-byte) units: at most 2 steps -- each unit is three loads, and
  // more, smaller blocks stream better (Qwen3-Next-shaped verify step: R 1 /
  // 2 / 3 / register-sized = 108 / 102 / 106 / 107 us)
  constexpr int cap = UB == 48 ? 2 : 4;
  return r < 1 ? 1 : (r > cap ? cap : r);
}

// Every (unit bytes, lanes per row, units per lane) pick_shape and
// gateup_shape return for rows of up to 8192 values.
#define PMOE_FOR_SHAPES_4(X)                                                     \
  X(32, 64, 1) X(32, 64, 2) X(16, 8, 1) X(16, 16, 1) X(16, 32, 1) X(16, 64, 1)   \
  X(16, 64, 2) X(16, 8, 3) X(16, 16, 3) X(16, 32, 3)
#define PMOE_FOR_SHAPES_6(X) X(48, 64, 1) X(48, 64, 2) X(48, 8, 1) X(48, 16, 1) X(48, 32, 1)
#define PMOE_FOR_SHAPES(BITS, X) \
  if constexpr (BITS == 4) {     \
    PMOE_FOR_SHAPES_4(X)         \
  } else {                       \
    PMOE_FOR_SHAPES_6(X)         \
  }

template <int BITS, bool DUAL>
int launch_qgemv(const GemvArgs& a, Shape sh, int max_experts, hipStream_t st) {
#define PMOE_CASE(U, L, G)                                                       \
  if (sh.ub == U && sh.lpr == L && sh.gpl == G) {                                \
    constexpr int R = rows_r<U, G, DUAL>();                                      \
    dim3 grid((a.rows_out + 4 * R * (64 / L) - 1) / (4 * R * (64 / L)), max_experts); \
    qgemv_kernel<U, L, G, R, DUAL><<<grid, 256, 0, st>>>(a);                     \
    PMOE_LAUNCH_CHECK("qgemv_kernel");                                           \
    return PMOE_OK;                                                              \
  }
  PMOE_FOR_SHAPES(BITS, PMOE_CASE)
#undef PMOE_CASE
  return fail(PMOE_EINVAL, "qgemv: unsupported row shape");
}

// One token: every block routes it itself.  Several: the router launch
// (router_route_kernel) has published the record.
template <int UB, int EPL, int L, int G>
int launch_gateup_routed(const GemvArgs& gu, const RouteDev& rt, int max_experts,
                         int32_t* inds_out, float* w_out, RouteRecord* rec, hipStream_t st) {
  constexpr int R = rows_r<UB, G, true>();
  constexpr int rows = 4 * R * (64 / L);
  dim3 grid((gu.rows_out + rows - 1) / rows, max_experts);
  if (rt.n == 1)
    gateup_routed_kernel<UB, L, G, R, EPL, false><<<grid, 256, 0, st>>>(gu, rt, inds_out, w_out,
                                                                        rec);
  else
    gateup_routed_kernel<UB, L, G, R, EPL, true><<<grid, 256, 0, st>>>(gu, rt, inds_out, w_out,
                                                                       rec);
  PMOE_LAUNCH_CHECK("gateup_routed_kernel");
  return PMOE_OK;
}

#ifndef PMOE_DOWN_SPLIT_MIN
#define PMOE_DOWN_SPLIT_MIN 17  // active-expert bound from which the down runs expert-split
#endif

template <int UB, int EPL, int L, int G>
int launch_down_routed(const GemvArgs& dn, const RouteDev& rt, int max_experts, uint16_t* out,
                       const RouteRecord* rec, hipStream_t st) {
  constexpr int R = rows_r<UB, G, false>();
  if (dn.out && max_experts >= PMOE_DOWN_SPLIT_MIN) {
    constexpr int rows = 4 * R * (64 / L);
    dim3 grid((dn.rows_out + rows - 1) / rows, max_experts);
    float* y = static_cast<float*>(dn.out);
    down_split_kernel<UB, L, G, R, EPL><<<grid, 256, 0, st>>>(dn, rt, y, rec);
    PMOE_LAUNCH_CHECK("down_split_kernel");
    dim3 cgrid((dn.rows_out + 255) / 256, rt.n);
    combine_y_kernel<<<cgrid, 256, 0, st>>>(y, rec, rt.kk, dn.rows_out, out);
    PMOE_LAUNCH_CHECK("combine_y_kernel");
    return PMOE_OK;
  }
  constexpr int T = R * (64 / L);
  const size_t lds = size_t(rt.n) * rt.kk * T * sizeof(float);
  if (lds > 48 * 1024) return fail(PMOE_EINVAL, "decode: too many rows per tile");
  dim3 grid((dn.rows_out + T - 1) / T);
  down_routed_kernel<UB, L, G, R, EPL><<<grid, 256, lds, st>>>(dn, rt, out, rec);
  PMOE_LAUNCH_CHECK("down_routed_kernel");
  return PMOE_OK;
}

// The router launch of a decode call: plain logits for one token, logits
// plus routing (router_route_kernel) for several.
template <int EPL>
int launch_router(const RouterIn& ri, const RouteDev& rt, RouteRecord* rec, const GemvArgs& gu,
                  int32_t* inds_out, float* w_out, hipStream_t st) {
  if (rt.n == 1)
    return router_logits_ext(ri.x, ri.w, ri.w_extra, ri.bias, rt.n, ri.d, rt.e, ri.out, st);
  PMOE_REQUIRE(ri.x && ri.w && ri.out && ri.arrive, "decode: null router input");
  PMOE_REQUIRE(ri.d % 8 == 0, "router_logits: hidden must be a multiple of 8");
  const int n = rt.n, n_w = rt.e;
  const int e = n_w + (ri.w_extra ? 1 : 0);
  RouteTail t{rt, rec, gu.table, gu.n_experts, gu.shared_slot, inds_out, w_out, ri.arrive};
  const bool full = ri.d % 512 == 0;
  ProfScope prof_scope(K_ROUTER_LOGITS, st);
  auto go = [&](auto tn, dim3 grid) {
    constexpr int TN = decltype(tn)::value;
    if (full)
      router_route_kernel<1, TN, 8, true, EPL><<<grid, 64 * kTailWaves, 0, st>>>(
          ri.x, ri.w, ri.w_extra, ri.bias, n, ri.d, e, n_w, ri.out, t);
    else
      router_route_kernel<1, TN, 8, false, EPL><<<grid, 64 * kTailWaves, 0, st>>>(
          ri.x, ri.w, ri.w_extra, ri.bias, n, ri.d, e, n_w, ri.out, t);
  };
  // Four tokens a wave, unless that leaves the launch under 64 blocks (few
  // experts: Qwen3-235B shapes at 8 tokens, 34 blocks), then two -- each
  // logit's arithmetic is the same either way (batch 8 133.8 -> 131.8 us;
  // two tokens a wave at 512 experts, 260 blocks, measured 79.4-80.0 against
  // 78.5-78.9 us for four).
  const int gx = (e + kTailWaves - 1) / kTailWaves;
  if (n >= 4 && gx * ((n + 3) / 4) >= 64)
    go(std::integral_constant<int, 4>{}, dim3(gx, (n + 3) / 4));
  else if (n >= 2)
    go(std::integral_constant<int, 2>{}, dim3(gx, (n + 1) / 2));
  else
    go(std::integral_constant<int, 1>{}, dim3(gx, n));
  PMOE_LAUNCH_CHECK("router_route_kernel");
  return PMOE_OK;
}

template <int BITS, int EPL>
int launch_routed(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt, int max_experts,
                  int32_t* inds_out, float* w_out, uint16_t* out, RouteRecord* rec,
                  hipStream_t st) {
  const Shape s1 = gateup_shape(BITS, gu, max_experts), s2 = pick_shape(BITS, dn.cols);
  int rc = PMOE_EINVAL;
  {
    ProfScope prof_scope(K_GATEUP, st);
#define PMOE_CASE(U, L, G)                                     \
  if (s1.ub == U && s1.lpr == L && s1.gpl == G)                 \
    rc = launch_gateup_routed<U, EPL, L, G>(gu, rt, max_experts, inds_out, w_out, rec, st);
    PMOE_FOR_SHAPES(BITS, PMOE_CASE)
#undef PMOE_CASE
  }
  if (rc == PMOE_EINVAL) return fail(PMOE_EINVAL, "decode: unsupported gate/up row shape");
  if (rc) return rc;
  rc = PMOE_EINVAL;
  {
    ProfScope prof_scope(K_DOWN, st);
#define PMOE_CASE(U, L, G)                     \
  if (s2.ub == U && s2.lpr == L && s2.gpl == G) \
    rc = launch_down_routed<U, EPL, L, G>(dn, rt, max_experts, out, rec, st);
    PMOE_FOR_SHAPES(BITS, PMOE_CASE)
#undef PMOE_CASE
  }
  if (rc == PMOE_EINVAL && pmoe_last_error()[0] == 0)
    return fail(PMOE_EINVAL, "decode: unsupported down row shape");
  return rc;
}

}  // namespace

Shape gateup_shape(int bits, const GemvArgs& gu, int) {
  const Shape half = pick_shape(bits, gu.cols, true);
  return half.ub == 16 && half.gpl > 2 ? pick_shape(bits, gu.cols) : half;
}

size_t decode_record_bytes() { return sizeof(RouteRecord); }

// One grouped projection launch (expert-major, dispatch in global memory).
int qgemv(const GemvArgs& a, int bits, bool dual, int max_experts, int, hipStream_t st) {
  PMOE_REQUIRE(a.cols % 64 == 0 && a.cols > 0, "qgemv: input dim must be a multiple of 64");
  const Shape sh = dual ? gateup_shape(bits, a, max_experts) : pick_shape(bits, a.cols);
  PMOE_REQUIRE(sh.lpr > 0, "qgemv: input dim too large (max 8192)");
  if (max_experts <= 0 || a.rows_out <= 0) return PMOE_OK;
  ProfScope prof_scope(dual ? K_GATEUP : K_DOWN, st);
  if (bits == 4)
    return dual ? launch_qgemv<4, true>(a, sh, max_experts, st)
                : launch_qgemv<4, false>(a, sh, max_experts, st);
  if (bits == 6)
    return dual ? launch_qgemv<6, true>(a, sh, max_experts, st)
                : launch_qgemv<6, false>(a, sh, max_experts, st);
  return fail(PMOE_EINVAL, "qgemv: bits must be 4 or 6");
}

// Decode MoE experts with routing fused into both projections: gate/up into
// gu.out (h), then down + combine into out [n, hidden].
int decode_route(const GemvArgs& gu, const RouteDev& rt, int32_t* inds_out, float* w_out,
                 void* record, const RouterIn& ri, hipStream_t st) {
  PMOE_REQUIRE(record != nullptr && inds_out != nullptr && w_out != nullptr,
               "decode: null routing outputs");
  PMOE_REQUIRE(rt.n >= 1 && rt.n * rt.kk <= kRouteMaxRows && rt.e + 1 <= kRouteMaxIds &&
                   rt.k <= kRouteMaxK && rt.k <= rt.e,
               "decode: bad routing shape");
  PMOE_REQUIRE(ri.x && ri.w && ri.out && ri.arrive, "decode: null router input");
  PMOE_REQUIRE(ri.d % 8 == 0, "router_logits: hidden must be a multiple of 8");
  RouteRecord* rec = static_cast<RouteRecord*>(record);
  const int epl = (rt.e + 63) / 64;
  const int n = rt.n, n_w = rt.e;
  const int e = n_w + (ri.w_extra ? 1 : 0);
  RouteTail t{rt, rec, gu.table, gu.n_experts, gu.shared_slot, inds_out, w_out, ri.arrive};
  const bool full = ri.d % 512 == 0;
  const int gx = (e + kTailWaves - 1) / kTailWaves;
  ProfScope prof_scope(K_ROUTER_LOGITS, st);
  auto go = [&](auto ep) {
    constexpr int EP = decltype(ep)::value;
    if (full)
      router_route_kernel<1, 1, 8, true, EP><<<dim3(gx, n), 64 * kTailWaves, 0, st>>>(
          ri.x, ri.w, ri.w_extra, ri.bias, n, ri.d, e, n_w, ri.out, t);
    else
      router_route_kernel<1, 1, 8, false, EP><<<dim3(gx, n), 64 * kTailWaves, 0, st>>>(
          ri.x, ri.w, ri.w_extra, ri.bias, n, ri.d, e, n_w, ri.out, t);
  };
  if (epl <= 2)
    go(std::integral_constant<int, 2>{});
  else if (epl <= 4)
    go(std::integral_constant<int, 4>{});
  else if (epl <= 8)
    go(std::integral_constant<int, 8>{});
  else if (epl <= 16)
    go(std::integral_constant<int, 16>{});
  else
    return fail(PMOE_EINVAL, "decode: too many experts");
  PMOE_LAUNCH_CHECK("router_route_kernel");
  return PMOE_OK;
}

int decode_routed(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt, int bits,
                  int32_t* inds_out, float* w_out, uint16_t* out, void* record,
                  const RouterIn& ri, hipStream_t st) {
  PMOE_REQUIRE(record != nullptr, "decode: null routing record");
  RouteRecord* rec = static_cast<RouteRecord*>(record);
  PMOE_REQUIRE(rt.n >= 1 && rt.n * rt.kk <= kRouteMaxRows, "decode: too many rows");
  PMOE_REQUIRE(rt.e + 1 <= kRouteMaxIds && rt.k <= kRouteMaxK && rt.k <= rt.e,
               "decode: bad experts/top-k");
  if (rt.scoring == PMOE_SCORE_SIGMOID)
    PMOE_REQUIRE(rt.e <= kRouteMaxSigE && rt.bias != nullptr && rt.n_group >= 1 &&
                     rt.n_group <= 64 && rt.e % rt.n_group == 0 && rt.topk_group >= 1 &&
                     rt.topk_group <= rt.n_group && rt.topk_group <= 8 &&
                     (rt.n_group == 1 || rt.e / rt.n_group >= 2) &&
                     rt.k <= (rt.e / rt.n_group) * rt.topk_group,
                 "decode: bad sigmoid group configuration");
  const int rows = rt.n * rt.kk;
  const int n_ids = rt.e + (rt.kk > rt.k ? 1 : 0);
  const int max_experts = rows < n_ids ? rows : n_ids;
  const int epl = (rt.e + 63) / 64;
  PMOE_REQUIRE(bits == 4 || bits == 6, "decode: bits must be 4 or 6");
#define PMOE_EPL(EP)                                                                     \
  if (epl <= EP) {                                                                       \
    const int rr = launch_router<EP>(ri, rt, rec, gu, inds_out, w_out, st);              \
    if (rr) return rr;                                                                   \
    if (bits == 4) return launch_routed<4, EP>(gu, dn, rt, max_experts, inds_out, w_out, out, rec, st); \
    return launch_routed<6, EP>(gu, dn, rt, max_experts, inds_out, w_out, out, rec, st); \
  }
  PMOE_EPL(2)
  PMOE_EPL(4)
  PMOE_EPL(8)
  PMOE_EPL(16)
#undef PMOE_EPL
  return fail(PMOE_EINVAL, "decode: too many experts");
}

}  // namespace pmoe

#ifdef PMOE_FUSED_TRACE
extern "C" int pmoe_debug_rtrace(uint64_t* out, int n) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(pmoe::g_rtrace), size_t(n) * sizeof(uint64_t)) ==
                 hipSuccess
             ? 0 : -2;
}
#endif
