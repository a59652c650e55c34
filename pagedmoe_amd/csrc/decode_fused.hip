// Fused decode layer: router logits -> routing -> gate/up + SwiGLU -> down +
// combine in ONE persistent launch.
//
// Replaces, for decode-sized batches, the same reference path as the
// three-launch decode in decode.hip: the router the reference taps
// (streaming.py:167-193), the selection (tests/test_stream.py:191-196;
// streaming.py:2424-2442), the slab path's three gather_qmm + SwiGLU
// (_run_slab, streaming.py:587-641) and the block's combine
// (tests/test_stream.py:198).
//
// The grid holds one 512-thread block per CU (all resident at once) and the
// phases are separated by two grid barriers:
//   A  router logits: one wave per logit row (expert), every token, in the
//      fixed summation order of router_logits_kernel (router.hip);
//      -> barrier 1
//   B  every block routes the batch from the logits with route_block
//      (route_common.h: bit-exact top-k, the same bits in every block);
//      block 0 publishes the routing outputs;
//   C  gate/up items (active expert, R rows) are dealt over all waves;
//      h = silu(g)*u is written as bf16.  Each wave then issues the weight
//      loads of its first down item;  -> barrier 2 (the down weights stream
//      in while the last gate/up rows finish)
//   D  block b owns hidden rows [b*T, b*T + T) of every active expert: its
//      waves run the down rows into LDS and the block combines them in fixed
//      k order (shared expert last), bf16 out.
// The GEMV arithmetic is the one of gemv_common.h, so the outputs are bit
// for bit those of the three-launch decode.
//
// Grid barrier protocol (DecodeSync: the first kDecodeSyncBytes of the
// workspace, all zero before the first call):
//   - every wave waits for its own memory operations (s_waitcnt 0), the
//     block syncs and thread 0 adds 1 to its group's counter (groups of
//     kDecodeGroup blocks, one 128-byte line each); the group's last block
//     resets that counter and adds 1 to arrive[i] -- device-scope atomics
//     on one address are serialised, so a flat counter of 256 arrivals
//     costs far more than two levels of 16;
//   - the block that brings arrive[i] to the group count resets it to 0 and
//     writes this launch's tag into every block's flag (one 128-byte line
//     per block); the others poll their own line, so no address is hot
//     while the weight stream saturates HBM;
//   - tags are 2*epoch+1 and 2*epoch+2; the last block at barrier 2 stores
//     epoch+1, so the next launch on the workspace waits for new tags
//     (no memset between launches: graph-safe).
// Data crossing a barrier (logits, h) is stored and loaded at device scope,
// which writes through / reads past the XCDs' L2s, so no cache writeback or
// invalidate is needed.  A poll that has waited its spin limit (0.5 s of the
// 100 MHz realtime clock by default; pmoe_set_barrier_spin) sets error bit 0
// of the workspace and gives up, so a launch always ends.  A block whose
// barrier-2 wait gave up, and every block that sees the error bit after
// barrier 2 (any block that gave up at barrier 1 set it before arriving
// there), writes NaN for its output rows instead of the combine, so a
// timed-out layer can never pass for a good one; the host reads the error
// word at its next sync point.
#ifdef PMOE_FUSED_TRACE
namespace pmoe { namespace { __device__ uint64_t g_trace[1024 * 32]; } }
#define PMOE_ROUTE_MARK(i) \
  do { if (threadIdx.x == 0) pmoe::g_trace[blockIdx.x * 32 + (i)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#endif
#include "gemv_common.h"
#include "pmoe_internal.h"
#include "pmoe_kernels.h"
#include "route_common.h"

#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

namespace pmoe {

namespace {

constexpr int kFWaves = 8;
constexpr int kXcds = 8;        // MI355X: blocks are dealt round robin over 8 XCDs
constexpr int kRouterXcds = 4;  // XCDs whose blocks compute the router logits
constexpr int kFThreads = 64 * kFWaves;
constexpr int kFMaxLogits = 8 * 1025;  // n * (E + shared gate) staged in LDS
constexpr int kFMaxTable = 1024;       // slot-table entries copied to LDS
constexpr int kFMaxH = 20480;          // bf16 h values staged in LDS in phase D
#ifndef PMOE_H_LDS
#define PMOE_H_LDS 1
#endif
constexpr uint64_t kSpinTicks = 50000000ull;  // 0.5 s at 100 MHz
uint64_t g_spin_ticks = kSpinTicks;           // host: limit passed to every launch
uint32_t g_split_probe = 0;                   // host: pmoe_set_split_probe
#ifndef PMOE_RANK1
#define PMOE_RANK1 1  // single-token routing by rank counts over the block
#endif
#ifndef PMOE_GU_PIPE
#define PMOE_GU_PIPE 1  // single-row gate/up items: two row steps in flight
#endif
#ifndef PMOE_POLL_SLEEP
#define PMOE_POLL_SLEEP 2  // s_sleep units (64 clocks) between two flag polls
#endif

struct FusedArgs {
  const uint16_t* x;           // [n, hidden]
  const uint16_t* gate_w;      // [E, hidden]
  const uint16_t* gate_extra;  // shared-expert gate row (logit column E) or null
  const float* logit_bias;     // [E] or null
  float* logits;               // [n, ld]
  GemvArgs gu, dn;
  uint16_t* out;               // [n, hidden]
  int32_t* inds_out;
  float* w_out;
  DecodeSync* sync;
  uint64_t spin;               // barrier poll limit, realtime-clock ticks
  uint32_t split_probe;        // debug: block 0 reports another XCD (placement check test)
  uint32_t round_y;            // given-ids launch: columns rounded to bf16 before the combine
  int n_blocks;
  int tile;                    // hidden rows per block in phase D
};

// Data that crosses a grid barrier (logits, h) is stored and loaded at
// device scope (sc1): stores write through the XCD's L2 and loads bypass
// its stale lines, so the barrier needs no cache writeback or invalidate.
constexpr bool kCoherentLoads = true;

#ifdef PMOE_FUSED_TRACE
// Debug builds: every block's thread 0 records realtime stamps per phase.
__device__ __forceinline__ void trace_mark(DecodeSync*, int i) {
  if (threadIdx.x == 0) g_trace[blockIdx.x * 32 + i] = __builtin_amdgcn_s_memrealtime();
}
#else
__device__ __forceinline__ void trace_mark(DecodeSync*, int) {}
#endif

// gemv_rows callback keeping step `sub`'s output in hv (each lane of a row
// group keeps a different step).
struct Collect {
  float* hv;
  int sub;
  __device__ __forceinline__ void operator()(int st, int, float v) const {
    if (sub == st) *hv = v;
  }
};
__device__ __forceinline__ Collect collect_fn(float& hv, int sub) { return Collect{&hv, sub}; }

template <class T>
__device__ __forceinline__ void shared_store(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block arrival + wait.  Every wave's stores (and loads) have completed
// before the block arrives.  Arrival is two-level, so no counter sees more
// than kDecodeGroup (or group-count) device-scope atomics: the last block of
// a group resets the group's counter and arrives at arrive[i]; the block
// that completes arrive[i] resets it and writes `tag` into every block's
// flag line; each block's thread 0 polls its own line (no shared hot spot
// while HBM is saturated).  Returns true (block-uniform) when this block's
// wait gave up after `spin` ticks.
__device__ __forceinline__ bool grid_barrier(DecodeSync* sy, int i, uint32_t tag,
                                             uint32_t n_blocks, uint64_t spin, int mark = -1) {
  __shared__ int s_last, s_gave_up;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's memory operations have completed
  __syncthreads();
  if (mark >= 0) trace_mark(nullptr, mark);
  uint8_t* base = reinterpret_cast<uint8_t*>(sy);
  if (threadIdx.x == 0) {
    const uint32_t g = blockIdx.x / kDecodeGroup;
    const uint32_t n_groups = (n_blocks + kDecodeGroup - 1) / kDecodeGroup;
    const uint32_t in_group = min(uint32_t(kDecodeGroup), n_blocks - g * kDecodeGroup);
    uint32_t* gc = reinterpret_cast<uint32_t*>(
        base + kDecodeGroupOffset + (size_t(i) * kDecodeMaxGroups + g) * kDecodeFlagStride);
    int last = 0;
    if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        in_group - 1) {
      if (mark >= 0) trace_mark(nullptr, 13);
      __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = __hip_atomic_fetch_add(&sy->arrive[i], 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == n_groups - 1;
      if (mark >= 0 && last) trace_mark(nullptr, 14);
    }
    s_last = last;
    s_gave_up = 0;
  }
  __syncthreads();
  uint8_t* flags = base + 256;
  if (s_last) {
    if (threadIdx.x == 0) {
      __hip_atomic_store(&sy->arrive[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (i == 1)  // every block has read the epoch by now
        __hip_atomic_store(&sy->epoch, tag >> 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    for (uint32_t b = threadIdx.x; b < n_blocks; b += blockDim.x)
      __hip_atomic_store(reinterpret_cast<uint32_t*>(flags + b * kDecodeFlagStride), tag,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if (threadIdx.x == 0) {
    const uint32_t* mine =
        reinterpret_cast<const uint32_t*>(flags + blockIdx.x * kDecodeFlagStride);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != tag) {
      __builtin_amdgcn_s_sleep(PMOE_POLL_SLEEP);
      if (__builtin_amdgcn_s_memrealtime() - t0 > spin) {
        __hip_atomic_fetch_or(&sy->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_gave_up = 1;
        break;
      }
    }
    if (mark >= 0) trace_mark(nullptr, 15);
  }
  __syncthreads();
  return s_gave_up != 0;
}

__device__ __forceinline__ void fma8(float& acc, const uint4& a, const uint4& b) {
  acc = __builtin_fmaf(bf16lo(a.x), bf16lo(b.x), acc);
  acc = __builtin_fmaf(bf16hi(a.x), bf16hi(b.x), acc);
  acc = __builtin_fmaf(bf16lo(a.y), bf16lo(b.y), acc);
  acc = __builtin_fmaf(bf16hi(a.y), bf16hi(b.y), acc);
  acc = __builtin_fmaf(bf16lo(a.z), bf16lo(b.z), acc);
  acc = __builtin_fmaf(bf16hi(a.z), bf16hi(b.z), acc);
  acc = __builtin_fmaf(bf16lo(a.w), bf16lo(b.w), acc);
  acc = __builtin_fmaf(bf16hi(a.w), bf16hi(b.w), acc);
}

// Logit (token t, row e) in router_logits_kernel's order: lane l owns
// d = 512p + 8l + j, fma over p then j, xor butterfly over the lanes; the
// bias is added to routed rows only.  The loads of 8 passes are issued
// together (one memory round trip for hidden <= 4096).  Every lane returns
// the logit.
// Dot of one router row with one token row over d columns, in the router's
// fixed lane order, 8 passes of 512 columns a group.  A group's loads are
// unconditional (passes and columns past the end re-read in-bounds data)
// and only the FMAs are guarded: with a guarded branch per pass, the
// compiler waited for the first passes' loads before issuing the later
// ones.
struct RouterGroup {
  uint4 w[8], x[8];
};

__device__ __forceinline__ void router_group_load(RouterGroup& g, const uint16_t* wrow,
                                                  const uint16_t* xrow, int d, int p0) {
  const int lane = threadIdx.x & 63;
  const int passes = (d + 511) / 512;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int col = min(min(p0 + j, passes - 1) * 512 + lane * 8, d - 8);
    g.w[j] = *reinterpret_cast<const uint4*>(wrow + col);
    g.x[j] = *reinterpret_cast<const uint4*>(xrow + col);
  }
}

__device__ __forceinline__ void router_group_fma(float& acc, const RouterGroup& g, int d,
                                                 int p0) {
  const int lane = threadIdx.x & 63;
  const int passes = (d + 511) / 512;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int col = (p0 + j) * 512 + lane * 8;
    if (p0 + j < passes && col < d) fma8(acc, g.x[j], g.w[j]);
  }
}

__device__ float router_row_dot(const uint16_t* wrow, const uint16_t* xrow, int d) {
  float acc = 0.0f;
  for (int p0 = 0; p0 < (d + 511) / 512; p0 += 8) {
    RouterGroup g;
    router_group_load(g, wrow, xrow, d, p0);
    router_group_fma(acc, g, d, p0);
  }
  return wave_sum_bfly(acc);
}

__device__ float router_dot(const FusedArgs& a, const RouteDev& rt, int e, int t) {
  const int d = a.gu.cols;
  const uint16_t* wrow = e < rt.e ? a.gate_w + size_t(e) * d : a.gate_extra;
  const float sum = router_row_dot(wrow, a.x + size_t(t) * d, d);
  return a.logit_bias && e < rt.e ? sum + a.logit_bias[e] : sum;
}

__device__ void router_pair(const FusedArgs& a, const RouteDev& rt, int e, int t) {
  const float v = router_dot(a, rt, e, t);
  if ((threadIdx.x & 63) == 0) shared_store(&a.logits[size_t(t) * rt.ld + e], v);
}

template <int UG, int LG, int GG, int RG, int UD, int LD, int GD, int RD, int EPL>
__global__ __launch_bounds__(kFThreads) void decode_fused_kernel(const FusedArgs a,
                                                                 const RouteDev rt) {
  __shared__ RouteLds L;
  __shared__ WaveTmp W[kFWaves];
  __shared__ int32_t s_rows[kFWaves][kRouteMaxRows];
  __shared__ __align__(16) float s_logit[kFMaxLogits];
  __shared__ int32_t s_slot[kRouteMaxRows];  // slot of active expert u
  __shared__ int32_t s_table[kFMaxTable];     // expert id -> slot, read at launch start
  __shared__ Rank1Lds R1;
  __shared__ uint4 s_h[kFMaxH / 8];           // phase D: h of the routed rows
  extern __shared__ float s_y[];             // [rows][tile]
  const int wave = threadIdx.x >> 6;
  const int lane_in_wave = threadIdx.x & 63;
  const int gw = blockIdx.x * kFWaves + wave;
  const int n_waves = a.n_blocks * kFWaves;
  DecodeSync* sy = a.sync;
  trace_mark(sy, 16);  // entry

  // this launch's barrier tags: 2*epoch + 1 and 2*epoch + 2 (never 0, the
  // initial flag value; consecutive launches differ)
  const uint32_t epoch = __hip_atomic_load(&sy->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t tag1 = 2u * epoch + 1u, tag2 = 2u * epoch + 2u;

  // the slot table comes in while the router runs (it is an input, not a
  // result of this launch), so the slots of the picked experts are LDS reads
  const bool table_lds = a.gu.n_experts <= kFMaxTable;
  if (table_lds)
    for (int i = threadIdx.x; i < a.gu.n_experts; i += kFThreads) s_table[i] = a.gu.table[i];

  // A: router logits on the blocks of the first kRouterXcds XCDs (block b
  // runs on XCD b % kXcds; a launch reaches the XCDs in turn, the last ~3 us
  // after the first), one (token, expert) pair per block before a block's
  // next wave takes one, so each CU streams only a few router rows.
  const int n_log = rt.e + (a.gate_extra ? 1 : 0);
  trace_mark(sy, 0);
  {
    const int n_pairs = n_log * rt.n;
    const int xcd = blockIdx.x % kXcds;
    auto on_xcd = [&](int x) { return (a.n_blocks - x + kXcds - 1) / kXcds; };
    int n_rblocks = 0, rank = -1;
    for (int x = 0; x < kRouterXcds; ++x) {
      if (x == xcd) rank = n_rblocks + int(blockIdx.x) / kXcds;
      n_rblocks += on_xcd(x);
    }
    if (rank >= 0) {
      for (int p = rank + n_rblocks * wave; p < n_pairs; p += n_rblocks * kFWaves) {
        const int t = p / n_log;
        router_pair(a, rt, p - t * n_log, t);
      }
    }
  }
  trace_mark(sy, 1);
  grid_barrier(sy, 0, tag1, a.n_blocks, a.spin);

  // B: routing (every block, identical bits)
  trace_mark(sy, 2);
  // the logits come in at device scope (written by other blocks), once
  for (int i = threadIdx.x; i < rt.n * rt.ld; i += kFThreads)
    s_logit[i] = __hip_atomic_load(rt.logits + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  trace_mark(sy, 9);
  RouteDev rl = rt;
  rl.logits = s_logit;
  static_assert(kFThreads >= 512, "route_rank1_select counts with 512 threads");
  const bool rank1 = PMOE_RANK1 && rank1_route_ok(rl);
  if (rank1)  // the weights follow before barrier 2 (route_rank1_weights)
    route_rank1_select(rl, s_logit, L, R1);
  else
    route_block<EPL, kFWaves>(rl, L, W, blockIdx.x == 0 ? a.inds_out : nullptr, a.w_out);
  trace_mark(sy, 3);
  const int rows = rt.n * rt.kk;
  const int n_act = L.n_active;
  for (int u = threadIdx.x; u < n_act; u += kFThreads) {
    const int e = L.active[u];
    s_slot[u] = e < a.gu.n_experts ? (table_lds ? s_table[e] : a.gu.table[e]) : a.gu.shared_slot;
  }
  __syncthreads();
  trace_mark(sy, 10);

  // C: gate/up + SwiGLU -> h.  An item's weights are held as two halves
  // (steps [0, RG/2) and [RG/2, RG)); on a wave's last item the weights of
  // its first down item are requested as each half is consumed, so the down
  // stream queues behind the gate/up stream instead of after it.
  constexpr int kHG = RG / 2;                 // steps per gate/up half
  constexpr int kRows = RG * (64 / LG);       // gate/up rows per item
  constexpr int kHD = RD > 1 ? RD / 2 : 1;    // steps per down half
  constexpr int kSub = RD * (64 / LD);        // down rows per item
  const int tile = a.tile;
  const int row0 = blockIdx.x * tile;
  const bool has_down = row0 < a.dn.rows_out;
  const int pre_slot = (has_down && wave < n_act) ? s_slot[wave] : -1;
  GemvRegs<UD, LD, GD, kHD, false> qd1, qd2;
  // (scheduling fences keep the loads where they are: hoisted above the
  // gate/up arithmetic they would hold both register sets at once)
  auto prefetch_down = [&](int half) {
    __builtin_amdgcn_sched_barrier(0);
    if (pre_slot >= 0) {
      if (half == 0) gemv_load<UD, LD, GD, kHD, false>(a.dn, pre_slot, row0, qd1);
      if (half == 1 && RD > 1)
        gemv_load<UD, LD, GD, kHD, false>(a.dn, pre_slot, row0 + kHD * (64 / LD), qd2);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  {
    const int chunks = (a.gu.rows_out + kRows - 1) / kRows;
    const int items = n_act * chunks;
    int cur = -1, m = 0;
    // item `it`; LAST: the wave's final item, which also issues the down
    // prefetch (peeled out of the loop so the prefetch registers are not
    // live across it)
    auto item = [&](int it, auto last_tag) {
      constexpr bool LAST = decltype(last_tag)::value;
      const int u = it / chunks;
      const int c = it - u * chunks;
      const int e = L.active[u];
      if (e != cur) {
        m = wave_rows_of(L, rows, e, s_rows[wave]);
        cur = e;
      }
      const int slot = s_slot[u];
      if (slot < 0) {  // not resident: phase D writes its zero rows
        if (LAST) {
          prefetch_down(0);
          prefetch_down(1);
        }
        return;
      }
      const int wrow0 = c * kRows;
      // h of one half (kHG steps) for activation row r: lane (rsub, sub)
      // keeps step sub's value, then one store instruction writes the
      // half's kHG * RPW consecutive bf16 (device-scope stores are written
      // through one by one: one instruction, not kHG, per half)
      const int g_sub = lane_in_wave % LG, g_rsub = lane_in_wave / LG;
      auto run_half = [&](auto& q, const GroupAct<UG>(&xa)[GG], int r, int hrow0) {
        float hv = 0.0f;
        gemv_rows<UG, LG, GG, kHG, true, Collect, true>(a.gu, q, xa, hrow0, collect_fn(hv, g_sub));
        const int o = hrow0 + g_sub * (64 / LG) + g_rsub;
        if (g_sub < kHG && o < a.gu.rows_out)
          shared_store(&static_cast<uint16_t*>(a.gu.out)[size_t(r) * a.gu.out_stride + o],
                       f2bf(hv));
      };
      GroupAct<UG> act[GG];
      int r = s_rows[wave][0];
      gemv_load_act<UG, LG, GG>(a.gu.act + size_t(r / rt.kk) * a.gu.act_stride, a.gu.cols, act);
      __builtin_amdgcn_sched_barrier(0);
      if (PMOE_GU_PIPE && m == 1) {
        // One activation row: the item's RG row steps go through a window of
        // two steps in flight, each step computed as soon as its words land.
        // (Issued all at once, a wave's loads come back in issue order but
        // are served in any order, so nearly every wave would receive its
        // last words at the end of the stream and do all its arithmetic
        // after it.)  Lane sub keeps step sub's value; one store writes the
        // item's RG * RPW bf16.
        constexpr int RPW = 64 / LG;
        GemvRegs<UG, LG, GG, 1, true> q[2];
        gemv_load<UG, LG, GG, 1, true>(a.gu, slot, wrow0, q[0]);
        gemv_load<UG, LG, GG, 1, true>(a.gu, slot, wrow0 + RPW, q[1]);
        float hv = 0.0f;
#pragma unroll
        for (int st = 0; st < RG; ++st) {
          __builtin_amdgcn_sched_barrier(0);
          gemv_rows<UG, LG, GG, 1, true, Collect, true>(a.gu, q[st & 1], act, wrow0 + st * RPW,
                                                        collect_fn(hv, g_sub - st));
          __builtin_amdgcn_sched_barrier(0);
          if (st + 2 < RG) gemv_load<UG, LG, GG, 1, true>(a.gu, slot, wrow0 + (st + 2) * RPW, q[st & 1]);
          if (LAST && st == kHG - 1) prefetch_down(0);
        }
        const int o = wrow0 + g_sub * RPW + g_rsub;
        if (g_sub < RG && o < a.gu.rows_out)
          shared_store(&static_cast<uint16_t*>(a.gu.out)[size_t(r) * a.gu.out_stride + o], f2bf(hv));
        if (LAST) prefetch_down(1);
        return;
      }
      GemvRegs<UG, LG, GG, kHG, true> qa, qb;
      gemv_load<UG, LG, GG, kHG, true>(a.gu, slot, wrow0, qa);
      gemv_load<UG, LG, GG, kHG, true>(a.gu, slot, wrow0 + kHG * (64 / LG), qb);
      __builtin_amdgcn_sched_barrier(0);
      for (int mi = 0; mi < m; ++mi) {
        if (mi > 0) {
          r = s_rows[wave][mi];
          gemv_load_act<UG, LG, GG>(a.gu.act + size_t(r / rt.kk) * a.gu.act_stride, a.gu.cols,
                                      act);
        }
        run_half(qa, act, r, wrow0);
      }
      if (LAST) prefetch_down(0);
      for (int mi = 0; mi < m; ++mi) {
        if (mi > 0 || m > 1) {
          r = s_rows[wave][mi];
          gemv_load_act<UG, LG, GG>(a.gu.act + size_t(r / rt.kk) * a.gu.act_stride, a.gu.cols,
                                      act);
        }
        run_half(qb, act, r, wrow0 + kHG * (64 / LG));
      }
      if (LAST) prefetch_down(1);
    };
    const int mine = gw < items ? (items - 1 - gw) / n_waves + 1 : 0;
    for (int j = 0; j + 1 < mine; ++j) item(gw + j * n_waves, std::false_type{});
    if (mine > 0) {
      item(gw + (mine - 1) * n_waves, std::true_type{});
    } else {
      prefetch_down(0);
      prefetch_down(1);
    }
  }
  trace_mark(sy, 7);
  if (rank1) route_rank1_weights(rl, s_logit, L, blockIdx.x == 0 ? a.inds_out : nullptr, a.w_out);
  trace_mark(sy, 4);
  __shared__ int s_poison;
  const bool late = grid_barrier(sy, 1, tag2, a.n_blocks, a.spin, 12);
  if (threadIdx.x == 0)
    s_poison = late || __hip_atomic_load(&sy->error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  trace_mark(sy, 5);

  // D: down rows of the block's tile into LDS, then the fixed-order combine
  if (has_down) {
    const int n_sub = tile / kSub;
    // h of every routed row comes in once per block (device scope, 16 bytes
    // a thread) when it fits, instead of once per row group of every wave
    const int hc = a.dn.cols / 8;  // 16-byte chunks per h row
    const bool h_lds = PMOE_H_LDS && rows * a.dn.cols <= kFMaxH;
    if (h_lds) {
      for (int i = threadIdx.x; i < rows * hc; i += kFThreads) {
        const int r = i / hc, c = i - r * hc;
        s_h[i] = load_act16<kCoherentLoads>(
            reinterpret_cast<const uint4*>(a.dn.act + size_t(r) * a.dn.act_stride) + c);
      }
      __syncthreads();
    }
    for (int u = wave; u < n_act; u += kFWaves) {
      const int e = L.active[u];
      const int m = wave_rows_of(L, rows, e, s_rows[wave]);
      const int slot = s_slot[u];
      for (int s = 0; s < n_sub; ++s) {
        const int wrow0 = row0 + s * kSub;
        if (slot < 0) {  // exact zero rows (streaming.py:715-719)
          for (int mi = 0; mi < m; ++mi)
            for (int t = threadIdx.x & 63; t < kSub; t += 64)
              s_y[s_rows[wave][mi] * tile + (wrow0 - row0) + t] = 0.0f;
          continue;
        }
        const int wrow1 = wrow0 + kHD * (64 / LD);
        if (u != wave || s != 0) {  // else prefetched in phase C
          gemv_load<UD, LD, GD, kHD, false>(a.dn, slot, wrow0, qd1);
          if (RD > 1) gemv_load<UD, LD, GD, kHD, false>(a.dn, slot, wrow1, qd2);
        }
        GroupAct<UD> act[GD];
        for (int mi = 0; mi < m; ++mi) {
          const int r = s_rows[wave][mi];
          if (h_lds)
            gemv_load_act<UD, LD, GD>(reinterpret_cast<const uint16_t*>(s_h) + size_t(r) * a.dn.cols,
                                      a.dn.cols, act);
          else
            gemv_load_act<UD, LD, GD, kCoherentLoads>(a.dn.act + size_t(r) * a.dn.act_stride,
                                                        a.dn.cols, act);
          auto to_lds = [&](int, int o, float v) { s_y[r * tile + (o - row0)] = v; };
          gemv_rows<UD, LD, GD, kHD, false>(a.dn, qd1, act, wrow0, to_lds);
          if (RD > 1) gemv_rows<UD, LD, GD, kHD, false>(a.dn, qd2, act, wrow1, to_lds);
        }
      }
      if (u == wave) trace_mark(sy, 11);
    }
    __syncthreads();
    trace_mark(sy, 8);
    const bool poison = s_poison != 0;
    for (int i = threadIdx.x; i < rt.n * tile; i += kFThreads) {
      const int n = i / tile, t = i - n * tile;
      const int o = row0 + t;
      if (o >= a.dn.rows_out) continue;
      float acc = 0.0f;
      for (int col = 0; col < rt.kk; ++col)
        acc = __builtin_fmaf(L.w[n * rt.kk + col], s_y[(n * rt.kk + col) * tile + t], acc);
      a.out[size_t(n) * a.dn.rows_out + o] = poison ? uint16_t(0x7fc0) : f2bf(acc);
    }
  }
  trace_mark(sy, 6);
}

// ------------------------------------------------- expert-per-XCD launch
//
// The same layer for one token with top-8 softmax routing (no shared
// expert), laid out so that each of the 8 picks is streamed by one block
// group: the blocks with b % 8 == x (group x) run pick x, the x-th expert of
// the top-8 list.  The dispatcher deals blocks round robin over the 8 XCDs
// (from wherever the previous dispatch left off), so a group shares one XCD
// and its L2.  Correctness depends on that: h travels through the group's L2
// (phase C).  Each block therefore checks its placement as it starts: it
// ORs the bit of its XCC_ID into its group's mask for this launch (a
// device-scope atomic; two masks alternate by launch parity, and the
// group's last arrival clears the other one for the next launch), and a
// block that finds another XCD's bit there sets error bit 1 at once and
// poisons its outputs; every h poll also gives up as soon as any error bit
// is set, so a split group fails loudly within microseconds instead of
// waiting out the spin limit.
//
// No phase waits at a barrier.  Everything one block needs from another
// travels as tagged data at device scope and is polled until the tag of
// this launch appears, so each block goes on the moment its own inputs
// exist:
//   A  every group computes all E logits, logit e by its wave e (the order
//      of router_logits_kernel, so every group gets the same bits), and
//      publishes each as a 64-bit word (tag << 32 | fp32 bits) into the
//      group's own logit array with a plain store, which stays in the
//      group's L2 (a device-scope store would first have to reach memory,
//      ~2 us at launch);
//   B  every block polls its group's E logit words into LDS and routes
//      (route_rank1_select: the same bits everywhere); slot of pick x;
//   C  the gate/up rows of pick x are dealt over the group's waves; h is
//      published as 32-bit words (tag & 0xFFFF << 16 | bf16) into the
//      group's L2 (plain stores; a group spread over two XCDs would never see
//      them and time out, loudly); each wave requests the weights of its
//      first down tile half way through its last gate/up item (requested
//      with its first rows, they lengthen the gate/up stream);
//   D  each block polls its group's h row into LDS; wave w of the group
//      computes down tile w (8 or 16 rows) of pick x into fp32 partial x,
//      then adds 1 to the tile's counter; the wave that brings it to a
//      multiple of 8 (the last of the 8 groups) reads the 8 partials and
//      writes acc = fma(w_x, y_x, acc) over x = 0..7 -- the order of the
//      grid-wide launch, so the outputs are bit for bit the same.
// The tag numbers the launch: thread 0 of every block adds 1 to its group's
// launch counter at entry, and counter / blocks-per-group (a power of two,
// so the sequence wraps cleanly) + 1 is the tag, the same in every block
// since all groups' counters advance alike.  Every launch rewrites every
// logit and h word (h of a non-resident pick as zeros), so a word's tag is
// at most one launch old and a 16-bit h tag cannot alias.  Tags make the
// exchange order-free: a word is taken when its tag matches, whenever it
// arrives.  A poll that has waited the spin limit sets error bit 0 and the
// block goes on poisoned: its h words and partial rows are NaN, which every
// output that depends on them inherits through the combine.
constexpr int kXcdPollSleep = 1;

// Router rows per wave in the group-local router: E <= this x waves per group.
constexpr int kXcdLogitsPerWave = 2;
// s_getreg operand of HW_REG_XCC_ID (hwreg 20), bits [3:0]: this wave's XCD.
constexpr int kHwRegXccId = 20 | (0 << 6) | ((4 - 1) << 11);

template <class T>
__device__ __forceinline__ T device_load(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Leading arguments: the pointers and sizes of the launch's first loads
// (launch counter, slot table, router rows, x), as plain arguments.  This
// file is built with kernel-argument preload, which puts a kernel's first
// argument dwords into SGPRs as its waves start, so those loads issue
// without waiting for the argument segment (a struct argument is not
// preloaded).
template <int UG, int LG, int GG, int RG, int UD, int LD, int GD, int RD>
__global__ __launch_bounds__(kFThreads) void decode_xcd_kernel(
    DecodeSync* sync_p, const int32_t* table_p, const uint16_t* x_p, const uint16_t* gate_p,
    const float* bias_p, int d, int n_experts, const FusedArgs a, const RouteDev rt) {
  constexpr int RPW = 64 / LG;
  constexpr int kRows = RG * RPW;           // gate/up rows per item
  constexpr int kHD = RD > 1 ? RD / 2 : 1;  // down steps per half
  constexpr int kSub = RD * (64 / LD);      // down rows per tile
  static_assert(kSub == 8 || kSub == 16, "down tiles of 8 or 16 rows");
  __shared__ RouteLds L;
  __shared__ Rank1Lds R1;
  __shared__ __align__(16) float s_logit[128];
  __shared__ int32_t s_table[128];
  __shared__ __align__(16) uint16_t s_h[kXcdMaxInter];
  __shared__ __align__(16) float s_y[kFWaves][kXcdCount][16];  // per wave: partial rows
  __shared__ uint32_t s_tag;
  __shared__ bool s_last, s_split;
  __shared__ int s_slot;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int xcd = blockIdx.x % kXcdCount;  // group
  const int per_xcd = a.n_blocks / kXcdCount;
  const int lw = (blockIdx.x / kXcdCount) * kFWaves + wave;  // wave index within the group
  const int n_lw = per_xcd * kFWaves;
  DecodeSync* sy = sync_p;
  uint8_t* hdr = reinterpret_cast<uint8_t*>(sy);
  uint64_t* lgx = reinterpret_cast<uint64_t*>(hdr + kXcdLogitOffset);
  uint32_t* hx = reinterpret_cast<uint32_t*>(hdr + kXcdHOffset) + size_t(xcd) * kXcdMaxInter;
  float* part = reinterpret_cast<float*>(hdr + kXcdPartOffset);
  const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();
  trace_mark(sy, 16);
#ifdef PMOE_FUSED_TRACE
  if (threadIdx.x == 0) {
    g_trace[blockIdx.x * 32 + 24] = __builtin_amdgcn_s_memtime();
    g_trace[blockIdx.x * 32 + 25] = __builtin_amdgcn_s_memrealtime();
  }
#endif
  // The slot table, the first group of this wave's router row and the
  // launch counter are requested at once; their values are used after the
  // router's FMAs, so their round trips overlap.  The row's loads go before
  // the counter's atomic (sched_barrier keeps that order): issued after it,
  // the compiler reused the atomic's return register for a row address and
  // waited for the atomic first.
  const int32_t tab = int(threadIdx.x) < n_experts ? table_p[threadIdx.x] : -1;
  RouterGroup rg0;
  if (lw < n_experts) router_group_load(rg0, gate_p + size_t(lw) * d, x_p, d, 0);
  __builtin_amdgcn_sched_barrier(0);
  uint32_t old = 0;
  if (threadIdx.x == 0)
    old = __hip_atomic_fetch_add(
        reinterpret_cast<uint32_t*>(hdr + kXcdCounterOffset + xcd * kDecodeFlagStride), 1u,
        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // A: every group computes all E logits (the router's fixed order, so each
  // group gets the same bits): the group's wave lw takes rows lw, lw + n_lw.
  // They are published after the barrier below into the group's own logit
  // words with plain stores, which land in the group's L2 where its polls
  // find them -- a device-scope store would have to reach memory before a
  // block on another XCD could see it, ~2 us at launch.
  trace_mark(sy, 0);
  if (int(threadIdx.x) < n_experts) s_table[threadIdx.x] = tab;  // the oldest load
  float lv[kXcdLogitsPerWave];
#pragma unroll
  for (int j = 0; j < kXcdLogitsPerWave; ++j) {
    const int e = lw + j * n_lw;
    lv[j] = 0.0f;
    if (e >= n_experts) break;
    float acc = 0.0f;
    for (int p0 = 0; p0 < (d + 511) / 512; p0 += 8) {
      RouterGroup g;
      if (j == 0 && p0 == 0)
        g = rg0;
      else
        router_group_load(g, gate_p + size_t(e) * d, x_p, d, p0);
      router_group_fma(acc, g, d, p0);
    }
    const float sum = wave_sum_bfly(acc);
    lv[j] = bias_p ? sum + bias_p[e] : sum;
  }
  if (threadIdx.x == 0) {
    s_tag = old / uint32_t(per_xcd) + 1u;
    s_last = old % uint32_t(per_xcd) == uint32_t(per_xcd) - 1u;
  }
  trace_mark(sy, 1);
  // only LDS crosses this barrier (slot table, tag): wave 0 does not wait
  // here for its logit store's device-scope acknowledgement (~1.2 us)
  block_lds_sync();
  const uint32_t tag = s_tag;
  uint64_t* lgx_g = lgx + size_t(xcd) * kXcdLogitStride;  // the group's logit words
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < kXcdLogitsPerWave; ++j) {
      const int e = lw + j * n_lw;
      if (e < n_experts) lgx_g[e] = (uint64_t(tag) << 32) | __float_as_uint(lv[j]);
    }
  }

  // placement: this block's XCD into the group's mask of this launch (the
  // atomic's answer is read after routing, so its round trip overlaps it)
  uint32_t xseen = 0, xbit = 0;
  if (threadIdx.x == 64) {
    uint32_t xcc = __builtin_amdgcn_s_getreg(kHwRegXccId) & 15u;
    if (a.split_probe && blockIdx.x == 0) xcc ^= 1u;
    xbit = 1u << xcc;
    uint32_t* masks = reinterpret_cast<uint32_t*>(hdr + kXcdCounterOffset +
                                                  xcd * kDecodeFlagStride) + 1;
    xseen = __hip_atomic_fetch_or(&masks[tag & 1u], xbit, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    if (s_last)
      __hip_atomic_store(&masks[(tag & 1u) ^ 1u], 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }

  // B: every logit of this launch into LDS (threads 128.. poll), then routing
  bool late = false;
  const int li = int(threadIdx.x) - 128;
  if (li >= 0 && li < rt.e) {
    while (true) {
      const uint64_t w = device_load(&lgx_g[li]);
      if (uint32_t(w >> 32) == tag) {
        s_logit[li] = __uint_as_float(uint32_t(w));
        break;
      }
      if (__builtin_amdgcn_s_memrealtime() - t_entry > a.spin) {
        late = true;
        break;
      }
      __builtin_amdgcn_s_sleep(kXcdPollSleep);
    }
  }
  const bool bad_logits = __syncthreads_or(late) != 0;
  trace_mark(sy, 2);
  RouteDev rl = rt;
  rl.logits = s_logit;
  route_rank1_select(rl, s_logit, L, R1);
  trace_mark(sy, 18);
  if (threadIdx.x == 0) {
    if (bad_logits)
      __hip_atomic_fetch_or(&sy->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int e = L.ids[xcd];  // always < rt.e: the ranks are a permutation
    s_slot = e >= 0 && e < rt.e ? s_table[e] : -1;
  }
  if (threadIdx.x == 64) {
    s_split = (xseen & ~xbit) != 0u;  // another XCD already ran a block of this group
    if (s_split)  // error bit 1: the group is split
      __hip_atomic_fetch_or(&sy->error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  trace_mark(sy, 3);
  const int slot = s_slot;
  const bool bad = bad_logits || s_split;

  // C: gate/up rows of the pick, two row steps in flight per wave (as in the
  // grid-wide launch's single-row items); h words carry the tag
  const uint32_t htag = (tag & 0xFFFFu) << 16;
  const int n_tiles = (a.dn.rows_out + kSub - 1) / kSub;
  const int pre_row = lw * kSub;
  const bool pre = slot >= 0 && lw < n_tiles;
  GemvRegs<UD, LD, GD, kHD, false> qd1, qd2;
  auto prefetch_down = [&](int half) {
    __builtin_amdgcn_sched_barrier(0);
    if (pre) {
      if (half == 0) gemv_load<UD, LD, GD, kHD, false>(a.dn, slot, pre_row, qd1);
      if (half == 1 && RD > 1)
        gemv_load<UD, LD, GD, kHD, false>(a.dn, slot, pre_row + kHD * (64 / LD), qd2);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  {
    const int items = (a.gu.rows_out + kRows - 1) / kRows;
    const int g_sub = lane % LG, g_rsub = lane / LG;
    // h stays in the group's XCD: a plain store lands in its L2 (and is
    // acknowledged there), where the group's device-scope reads find it
    auto put_h = [&](int o, float hv) {
      const uint32_t bits = bad ? 0x7fc0u : (slot < 0 ? 0u : uint32_t(f2bf(hv)));
      hx[o] = htag | bits;
    };
    GroupAct<UG> act[GG];
    if (slot >= 0 && lw < items) gemv_load_act<UG, LG, GG>(a.gu.act, a.gu.cols, act);
    auto item = [&](int it, auto last_tag) {
      constexpr bool LAST = decltype(last_tag)::value;
      const int wrow0 = it * kRows;
      const int o = wrow0 + g_sub * RPW + g_rsub;
      if (slot < 0) {  // not resident: this launch's h words are zeros
        if (g_sub < RG && o < a.gu.rows_out) put_h(o, 0.0f);
        return;
      }
      GemvRegs<UG, LG, GG, 1, true> q[2];
      gemv_load<UG, LG, GG, 1, true>(a.gu, slot, wrow0, q[0]);
      gemv_load<UG, LG, GG, 1, true>(a.gu, slot, wrow0 + RPW, q[1]);
      float hv = 0.0f;
#pragma unroll
      for (int st = 0; st < RG; ++st) {
        __builtin_amdgcn_sched_barrier(0);
        gemv_rows<UG, LG, GG, 1, true, Collect, true>(a.gu, q[st & 1], act, wrow0 + st * RPW,
                                                      collect_fn(hv, g_sub - st));
        __builtin_amdgcn_sched_barrier(0);
        if (st + 2 < RG) gemv_load<UG, LG, GG, 1, true>(a.gu, slot, wrow0 + (st + 2) * RPW, q[st & 1]);
        if (LAST && st == RG / 2 - 1) prefetch_down(0);
      }
      if (g_sub < RG && o < a.gu.rows_out) put_h(o, hv);
      if (LAST) prefetch_down(1);
    };
    const int mine = lw < items ? (items - 1 - lw) / n_lw + 1 : 0;
    for (int j = 0; j + 1 < mine; ++j) item(lw + j * n_lw, std::false_type{});
    if (mine > 0) {
      item(lw + (mine - 1) * n_lw, std::true_type{});
    } else {
      prefetch_down(0);
      prefetch_down(1);
    }
  }
  trace_mark(sy, 7);

  // D: the group's h row into LDS (every word of this launch), then the down
  // tiles of the pick and the combine
  bool poison = bad;
  if (slot >= 0) {
    // 4 words a thread per poll (one 16-byte load, two 8-byte device-scope
    // reads); a chunk is kept once all 4 carry this launch's tag
    bool h_late = false;
    for (int c = threadIdx.x; c < a.dn.cols / 4; c += kFThreads) {
      const uint64_t* src = reinterpret_cast<const uint64_t*>(hx) + 2 * c;
      while (true) {
        const uint64_t w0 = device_load(src), w1 = device_load(src + 1);
        const uint32_t t = uint32_t(w0) & uint32_t(w0 >> 32) & uint32_t(w1) & uint32_t(w1 >> 32);
        const uint32_t u = uint32_t(w0) | uint32_t(w0 >> 32) | uint32_t(w1) | uint32_t(w1 >> 32);
        if ((t & 0xFFFF0000u) == htag && (u & 0xFFFF0000u) == htag) {
          *reinterpret_cast<uint2*>(&s_h[4 * c]) =
              make_uint2((uint32_t(w0) & 0xFFFFu) | (uint32_t(w0 >> 32) << 16),
                         (uint32_t(w1) & 0xFFFFu) | (uint32_t(w1 >> 32) << 16));
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t_entry > a.spin ||
            device_load(&sy->error) != 0u) {  // timed out, or another block failed
          h_late = true;
          break;
        }
        __builtin_amdgcn_s_sleep(kXcdPollSleep);
      }
    }
    if (__syncthreads_or(h_late)) {
      poison = true;
      if (threadIdx.x == 0)
        __hip_atomic_fetch_or(&sy->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  trace_mark(sy, 8);
  const float kNaN = __uint_as_float(0x7fc00000u);
  float* yx = part + size_t(xcd) * kXcdMaxHidden;
  constexpr int kQ = kSub / 4;  // 16-byte chunks of a tile
  for (int tl = lw; tl < n_tiles; tl += n_lw) {
    const int row0 = tl * kSub;
    float* own = s_y[wave][xcd];
    if (slot < 0) {  // not resident: exact zero rows (streaming.py:715-719)
      if (lane < kSub) own[lane] = poison ? kNaN : 0.0f;
    } else {
      if (tl != lw) {
        gemv_load<UD, LD, GD, kHD, false>(a.dn, slot, row0, qd1);
        if (RD > 1) gemv_load<UD, LD, GD, kHD, false>(a.dn, slot, row0 + kHD * (64 / LD), qd2);
      }
      GroupAct<UD> act[GD];
      gemv_load_act<UD, LD, GD>(s_h, a.dn.cols, act);
      auto to_own = [&](int, int o, float v) { own[o - row0] = poison ? kNaN : v; };
      gemv_rows<UD, LD, GD, kHD, false>(a.dn, qd1, act, row0, to_own);
      if (RD > 1) gemv_rows<UD, LD, GD, kHD, false>(a.dn, qd2, act, row0 + kHD * (64 / LD), to_own);
    }
    wave_lds_sync();
    trace_mark(sy, 11);
    // rows past rows_out are never read: a tile's partial is stored whole
    if (lane < kQ)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(yx + row0) + 2 * lane,
                         *reinterpret_cast<const uint64_t*>(own + 4 * lane), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT),
      __hip_atomic_store(reinterpret_cast<uint64_t*>(yx + row0) + 2 * lane + 1,
                         *reinterpret_cast<const uint64_t*>(own + 4 * lane + 2), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the partial has reached device scope
    uint32_t old = 0;
    if (lane == 0)
      old = __hip_atomic_fetch_add(
          reinterpret_cast<uint32_t*>(hdr + kXcdTileOffset + size_t(tl) * kXcdTileStride), 1u,
          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    trace_mark(sy, 19);
    if (old % kXcdCount != kXcdCount - 1) continue;
    // last of the 8: the other groups' partials of the tile into LDS
    if (lane < kXcdCount * kQ) {
      const int x = lane / kQ, c = lane % kQ;
      if (x != xcd) {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(
            part + size_t(x) * kXcdMaxHidden + row0 + 4 * c);
        *reinterpret_cast<uint64_t*>(&s_y[wave][x][4 * c]) = device_load(src);
        *reinterpret_cast<uint64_t*>(&s_y[wave][x][4 * c + 2]) = device_load(src + 1);
      }
    }
    wave_lds_sync();
    trace_mark(sy, 20);
    // the combine weights of the picks, as route_rank1_weights computes them
    const int k = rt.k;
    const int ik = lane < k ? L.ids[lane] : 0;
    const float pv = lane < k ? s_logit[ik] : 0.0f;
    const float m = lane_value(pv, 0);
    const float ej = lane < k ? pexp(pv - m) : 0.0f;
    float ssum = 0.0f;
    for (int j = 0; j < k; ++j) ssum = ssum + lane_value(ej, j);
    const float wk = ej / ssum;
    const int o = row0 + lane;
    if (lane < kSub && o < a.dn.rows_out) {
      float acc = 0.0f;
#pragma unroll
      for (int x = 0; x < kXcdCount; ++x) acc = __builtin_fmaf(lane_value(wk, x), s_y[wave][x][lane], acc);
      a.out[o] = f2bf(acc);
    }
  }
  // the routing outputs, off the critical path
  if (blockIdx.x == 0) route_rank1_weights(rl, s_logit, L, a.inds_out, a.w_out);
  trace_mark(sy, 6);
#ifdef PMOE_FUSED_TRACE
  if (threadIdx.x == 0) {
    g_trace[blockIdx.x * 32 + 26] = __builtin_amdgcn_s_memtime();
    g_trace[blockIdx.x * 32 + 27] = __builtin_amdgcn_s_memrealtime();
  }
#endif
}

// The experts of one token given its 8 ids and weights (pmoe_moe_experts),
// expert per XCD as above without the router: group x = blockIdx % 8 runs
// column x (ids[x], slot table[ids[x]]; an id outside [0, E) is dropped,
// a non-resident one gives zero rows) -- gate/up + SwiGLU, h exchanged in
// the group's L2, down rows.  A shared expert is split over the groups:
// group x computes gate/up rows [x*R, x*R + R) of it first (h as
// launch-tagged 64-bit words at device scope, which every group reads) and
// its down tiles t with t % 8 == x (launch-tagged 64-bit words at device
// scope).  Each column's down rows are rounded to bf16, as the three-launch
// path's per-slot outputs are (round_y; the decode block combines fp32 rows);
// the last of a tile's 8 group arrivals combines it in column order with
// fp32 fmas, the shared expert last with weight 1 -- the three-launch path's
// outputs bit for bit.
//
// The launch tag comes from the group's launch counter (thread 0); it is
// needed from the first h store on, so the block waits for it once, after
// its first item's weights are requested.  A CU's vector memory requests
// return in order: the h polls are answered once the down weights requested
// during the last gate/up item have landed, and that request overlaps the
// exchange.
template <int UG, int LG, int GG, int RG, int UD, int LD, int GD, int RD>
__global__ __launch_bounds__(kFThreads) void experts_xcd_kernel(
    DecodeSync* sync_p, const int32_t* ids_p, const float* w_p, int n_experts, int shared_slot,
    const FusedArgs a) {
  constexpr int RPW = 64 / LG;
  constexpr int kRows = RG * RPW;           // gate/up rows per item
  constexpr int kHD = RD > 1 ? RD / 2 : 1;  // down steps per half
  constexpr int kSub = RD * (64 / LD);      // down rows per tile
  static_assert(kSub == 8 || kSub == 16, "down tiles of 8 or 16 rows");
  __shared__ __align__(16) uint16_t s_h[kXcdMaxInter];   // the column's h
  __shared__ __align__(16) uint16_t s_hs[kXcdMaxInter];  // the shared expert's h
  __shared__ __align__(16) float s_y[kFWaves][kXcdCount + 1][16];
  __shared__ uint32_t s_tag;
  __shared__ bool s_last;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int xcd = blockIdx.x % kXcdCount;
  const int per_xcd = a.n_blocks / kXcdCount;
  const int lw = (blockIdx.x / kXcdCount) * kFWaves + wave;
  const int n_lw = per_xcd * kFWaves;
  DecodeSync* sy = sync_p;
  uint8_t* hdr = reinterpret_cast<uint8_t*>(sy);
  // the column's h: (tag & 0xFFFF) << 16 | bf16 words in the group's L2
  uint32_t* hx = reinterpret_cast<uint32_t*>(hdr + kXcdEHOffset) + size_t(xcd) * kXcdMaxInter;
  uint64_t* hs = reinterpret_cast<uint64_t*>(hdr + kXcdSharedHOffset);
  float* part = reinterpret_cast<float*>(hdr + kXcdEPartOffset);
  uint64_t* ps = reinterpret_cast<uint64_t*>(hdr + kXcdSharedPartOffset);
  uint32_t* line = reinterpret_cast<uint32_t*>(hdr + kXcdCounterOffset + xcd * kDecodeFlagStride);
  const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();
  trace_mark(sy, 16);
  // the launch counter first: its answer (the tag) is waited for after the
  // first item's weight loads are issued
  uint32_t old = 0;
  if (threadIdx.x == 0)
    old = __hip_atomic_fetch_add(&line[kXcdECounterWord], 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_sched_barrier(0);
#ifdef PMOE_FUSED_TRACE
  if (threadIdx.x == 0) {
    asm volatile("" ::"v"(old));
    trace_mark(sy, 22);  // the launch count is back
  }
#endif
  const bool has_shared = shared_slot >= 0;
  // the column's id and slot, the same for the whole block, read once
  // through the scalar cache (as constant memory: neither is written during
  // the launch): as vector loads the two dependent reads queued behind
  // every wave's activation loads and the slot was known 5-7 us into the
  // launch
  typedef const __attribute__((address_space(4))) int32_t ConstI32;
  const int col_id = *(ConstI32*)(ids_p + xcd);
  const int col_slot = col_id >= 0 && col_id < n_experts ? *(ConstI32*)(a.gu.table + col_id) : -1;
  auto load_slot = [&]() { return col_slot; };

  const int inter = a.gu.rows_out;
  const int sh_rows =
      has_shared ? ((inter + kXcdCount - 1) / kXcdCount + kRows - 1) / kRows * kRows : 0;
  const int sr0 = xcd * sh_rows, sr1 = min(inter, sr0 + sh_rows);
  const int n_sh = sr1 > sr0 ? (sr1 - sr0 + kRows - 1) / kRows : 0;  // shared items, first
  const int items = n_sh + (inter + kRows - 1) / kRows;
  const int n_tiles = (a.dn.rows_out + kSub - 1) / kSub;
  // down items: this group's shared tiles (t % 8 == xcd) first, then every tile
  const int n_sh_t = has_shared ? (n_tiles - xcd + kXcdCount - 1) / kXcdCount : 0;
  const int n_dt = n_sh_t + n_tiles;
  auto d_tile = [&](int j) { return j < n_sh_t ? j * kXcdCount + xcd : j - n_sh_t; };

  uint32_t tag = 0, htag = 0, xseen = 0, xbit = 0;
  auto sync_tag = [&]() {
    if (threadIdx.x == 0) {
      // opaque: the division stays here, after the first item's weight
      // loads, instead of being hoisted to the kernel's head, where its wait
      // for the count also waited for the activation loads
      asm volatile("" : "+v"(old));
      s_tag = old / uint32_t(per_xcd) + 1u;
      s_last = old % uint32_t(per_xcd) == uint32_t(per_xcd) - 1u;
    }
    block_lds_sync();
    tag = s_tag;
    htag = (tag & 0xFFFFu) << 16;
    trace_mark(sy, 0);
    // placement: this block's XCD into the group's mask of this launch (its
    // answer is read after the h polls); the group's last block clears the
    // other mask for the next launch
    if (threadIdx.x == 64) {
      uint32_t xcc = __builtin_amdgcn_s_getreg(kHwRegXccId) & 15u;
      if (a.split_probe && blockIdx.x == 0) xcc ^= 1u;
      xbit = 1u << xcc;
      xseen = __hip_atomic_fetch_or(&line[kXcdECounterWord + 1 + int(tag & 1u)], xbit,
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (s_last)
        __hip_atomic_store(&line[kXcdECounterWord + 1 + int((tag & 1u) ^ 1u)], 0u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  // the wave's first down item, requested during its last gate/up item
  GemvRegs<UD, LD, GD, kHD, false> qd1, qd2;
  auto prefetch_down = [&](int half) {
    __builtin_amdgcn_sched_barrier(0);
    if (lw < n_dt) {
      int pslot;
      if (lw < n_sh_t)
        pslot = shared_slot;
      else
        pslot = load_slot();
      const int prow = d_tile(lw) * kSub;
      if (pslot >= 0) {
        if (half == 0) gemv_load<UD, LD, GD, kHD, false>(a.dn, pslot, prow, qd1);
        if (half == 1 && RD > 1)
          gemv_load<UD, LD, GD, kHD, false>(a.dn, pslot, prow + kHD * (64 / LD), qd2);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  {
    const int g_sub = lane % LG, g_rsub = lane / LG;
    // the token's activations, loaded by the wave's first item after its
    // weights are requested (waiting for them first would hold the weights
    // back by a round trip)
    GroupAct<UG> act[GG];
    auto item = [&](int it, bool first, auto last_tag) {
      constexpr bool LAST = decltype(last_tag)::value;
      const bool sh = it < n_sh;
      const int wrow0 = sh ? sr0 + it * kRows : (it - n_sh) * kRows;
      const int rlim = sh ? sr1 : inter;
      int islot;
      if (sh)
        islot = shared_slot;
      else
        islot = load_slot();
      const int o = wrow0 + g_sub * RPW + g_rsub;
      if (islot < 0) {  // a column that is not resident: zero h words
        if (first) sync_tag();
        if (g_sub < RG && o < rlim) hx[o] = htag;
        if (LAST) {
          prefetch_down(0);
          prefetch_down(1);
        }
        return;
      }
#ifdef PMOE_FUSED_TRACE
      if (first && threadIdx.x == 0) {
        asm volatile("" ::"v"(islot));
        trace_mark(sy, 23);  // the first item's slot is known
      }
#endif
      GemvRegs<UG, LG, GG, 1, true> q[2];
      gemv_load<UG, LG, GG, 1, true>(a.gu, islot, wrow0, q[0]);
      gemv_load<UG, LG, GG, 1, true>(a.gu, islot, wrow0 + RPW, q[1]);
      __builtin_amdgcn_sched_barrier(0);
      if (first) {
        trace_mark(sy, 24);  // its weights are requested
        gemv_load_act<UG, LG, GG>(a.gu.act, a.gu.cols, act);
        __builtin_amdgcn_sched_barrier(0);
        sync_tag();
      }
      float hv = 0.0f;
#pragma unroll
      for (int st = 0; st < RG; ++st) {
        __builtin_amdgcn_sched_barrier(0);
        gemv_rows<UG, LG, GG, 1, true, Collect, true>(a.gu, q[st & 1], act, wrow0 + st * RPW,
                                                      collect_fn(hv, g_sub - st));
        __builtin_amdgcn_sched_barrier(0);
        if (st + 2 < RG)
          gemv_load<UG, LG, GG, 1, true>(a.gu, islot, wrow0 + (st + 2) * RPW, q[st & 1]);
        if (LAST && st == RG / 2 - 1) prefetch_down(0);
      }
      if (first) trace_mark(sy, 21);
      if (g_sub < RG && o < rlim) {
        const uint32_t bits = uint32_t(f2bf(hv));
        if (sh)  // every group reads the shared expert's h
          __hip_atomic_store(&hs[o], (uint64_t(tag) << 32) | bits, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        else  // the column's h stays in the group's L2
          hx[o] = htag | bits;
      }
      if (LAST) prefetch_down(1);
    };
    const int mine = lw < items ? (items - 1 - lw) / n_lw + 1 : 0;
    for (int j = 0; j + 1 < mine; ++j) item(lw + j * n_lw, j == 0, std::false_type{});
    if (mine > 0) {
      item(lw + (mine - 1) * n_lw, mine == 1, std::true_type{});
    } else {
      sync_tag();
      prefetch_down(0);
      prefetch_down(1);
    }
  }
  trace_mark(sy, 7);

  // D: h rows into LDS -- the column's (the group's L2) and, for blocks with
  // a shared tile, the shared expert's (device scope)
  bool h_late = false;
  auto timed_out = [&]() {
    return __builtin_amdgcn_s_memrealtime() - t_entry > a.spin || device_load(&sy->error) != 0u;
  };
  const int slot = load_slot();
  if (slot >= 0) {
    for (int c = threadIdx.x; c < a.dn.cols / 4 && !h_late; c += kFThreads) {
      const uint64_t* src = reinterpret_cast<const uint64_t*>(hx) + 2 * c;
      while (true) {
        const uint64_t w0 = device_load(src), w1 = device_load(src + 1);
        const uint32_t t = uint32_t(w0) & uint32_t(w0 >> 32) & uint32_t(w1) & uint32_t(w1 >> 32);
        const uint32_t u = uint32_t(w0) | uint32_t(w0 >> 32) | uint32_t(w1) | uint32_t(w1 >> 32);
        if ((t & 0xFFFF0000u) == htag && (u & 0xFFFF0000u) == htag) {
          *reinterpret_cast<uint2*>(&s_h[4 * c]) =
              make_uint2((uint32_t(w0) & 0xFFFFu) | (uint32_t(w0 >> 32) << 16),
                         (uint32_t(w1) & 0xFFFFu) | (uint32_t(w1 >> 32) << 16));
          break;
        }
        if (timed_out()) {
          h_late = true;
          break;
        }
        __builtin_amdgcn_s_sleep(kXcdPollSleep);
      }
    }
  }
  if (has_shared && (blockIdx.x / kXcdCount) * kFWaves < n_sh_t) {
    for (int c = threadIdx.x; c < a.dn.cols / 2 && !h_late; c += kFThreads) {
      while (true) {
        const uint64_t w0 = device_load(&hs[2 * c]), w1 = device_load(&hs[2 * c + 1]);
        if (uint32_t(w0 >> 32) == tag && uint32_t(w1 >> 32) == tag) {
          *reinterpret_cast<uint32_t*>(&s_hs[2 * c]) =
              (uint32_t(w0) & 0xFFFFu) | (uint32_t(w1) << 16);
          break;
        }
        if (timed_out()) {
          h_late = true;
          break;
        }
        __builtin_amdgcn_s_sleep(kXcdPollSleep);
      }
    }
  }
  bool split = false;
  if (threadIdx.x == 64 && (xseen & ~xbit) != 0u) {  // another XCD ran a block of this group
    split = true;
    __hip_atomic_fetch_or(&sy->error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  bool poison = false;
  if (__syncthreads_or(h_late || split)) {
    poison = true;
    if (threadIdx.x == 0)
      __hip_atomic_fetch_or(&sy->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  trace_mark(sy, 8);

  const float kNaN = __uint_as_float(0x7fc00000u);
  float* yx = part + size_t(xcd) * kXcdMaxHidden;
  constexpr int kQ = kSub / 4;  // 16-byte chunks of a tile
  // the combine's inputs: column weights and which columns count
  const int idc = lane < kXcdCount ? ids_p[lane] : -1;
  const float wc = lane < kXcdCount ? w_p[lane] : 0.0f;
  const uint64_t kept = wave_ballot(idc >= 0 && idc < n_experts);
  for (int j = lw; j < n_dt; j += n_lw) {
    const bool sh = j < n_sh_t;
    const int tl = d_tile(j);
    const int row0 = tl * kSub;
    const int dslot = sh ? shared_slot : slot;
    float* own = s_y[wave][xcd];
    if (dslot < 0) {  // not resident: exact zero rows
      if (lane < kSub) own[lane] = poison ? kNaN : 0.0f;
    } else {
      if (j != lw) {
        gemv_load<UD, LD, GD, kHD, false>(a.dn, dslot, row0, qd1);
        if (RD > 1) gemv_load<UD, LD, GD, kHD, false>(a.dn, dslot, row0 + kHD * (64 / LD), qd2);
      }
      GroupAct<UD> act[GD];
      gemv_load_act<UD, LD, GD>(sh ? s_hs : s_h, a.dn.cols, act);
      // each column's output as the bf16 the per-slot outputs hold (or the
      // fp32 value, for the decode block's combine)
      auto to_own = [&](int, int o, float v) {
        own[o - row0] = poison ? kNaN : (a.round_y ? bf16f(f2bf(v)) : v);
      };
      gemv_rows<UD, LD, GD, kHD, false>(a.dn, qd1, act, row0, to_own);
      if (RD > 1) gemv_rows<UD, LD, GD, kHD, false>(a.dn, qd2, act, row0 + kHD * (64 / LD), to_own);
    }
    wave_lds_sync();
    trace_mark(sy, 11);
    if (sh) {  // the shared rows of this tile, for whichever group combines it
      if (lane < kSub)
        __hip_atomic_store(&ps[row0 + lane], (uint64_t(tag) << 32) | __float_as_uint(own[lane]),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    // rows past rows_out are never read: a tile's partial is stored whole
    if (lane < kQ)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(yx + row0) + 2 * lane,
                         *reinterpret_cast<const uint64_t*>(own + 4 * lane), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT),
      __hip_atomic_store(reinterpret_cast<uint64_t*>(yx + row0) + 2 * lane + 1,
                         *reinterpret_cast<const uint64_t*>(own + 4 * lane + 2), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the partial has reached device scope
    uint32_t prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(
          reinterpret_cast<uint32_t*>(hdr + kXcdTileOffset + size_t(tl) * kXcdTileStride), 1u,
          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    trace_mark(sy, 19);
    if (prev % kXcdCount != kXcdCount - 1) continue;
    // last of the 8: the other groups' rows of the tile (and the shared
    // rows) into LDS
    if (lane < kXcdCount * kQ) {
      const int x = lane / kQ, c = lane % kQ;
      if (x != xcd) {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(
            part + size_t(x) * kXcdMaxHidden + row0 + 4 * c);
        *reinterpret_cast<uint64_t*>(&s_y[wave][x][4 * c]) = device_load(src);
        *reinterpret_cast<uint64_t*>(&s_y[wave][x][4 * c + 2]) = device_load(src + 1);
      }
    }
    bool s_bad = false;
    if (has_shared && lane < kSub) {
      while (true) {
        const uint64_t w = device_load(&ps[row0 + lane]);
        if (uint32_t(w >> 32) == tag) {
          s_y[wave][kXcdCount][lane] = __uint_as_float(uint32_t(w));
          break;
        }
        if (timed_out()) {
          s_bad = true;
          break;
        }
        __builtin_amdgcn_s_sleep(kXcdPollSleep);
      }
    }
    if (wave_ballot(s_bad) != 0ull && lane == 0)
      __hip_atomic_fetch_or(&sy->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wave_lds_sync();
    trace_mark(sy, 20);
    const int o = row0 + lane;
    if (lane < kSub && o < a.dn.rows_out) {
      float acc = 0.0f;
#pragma unroll
      for (int x = 0; x < kXcdCount; ++x)
        if ((kept >> x) & 1ull) acc = __builtin_fmaf(lane_value(wc, x), s_y[wave][x][lane], acc);
      if (has_shared) acc = __builtin_fmaf(1.0f, s_y[wave][kXcdCount][lane], acc);
      a.out[o] = s_bad ? f2bf(kNaN) : f2bf(acc);
    }
  }
  trace_mark(sy, 6);
}

// ---------------------------------------------------------------- host side

// Row steps per wave item: weights of one item stay in registers next to the
// activations, within the 256 VGPRs of two waves per SIMD.
template <int UB, int GPL, bool DUAL>
constexpr int fused_r(int cap) {
  constexpr int per_step = GPL * (Unit<UB>::kWords + 2) * (DUAL ? 2 : 1);
  constexpr int budget = 180 - GPL * (Unit<UB>::kVals / 2 + 1);
  int r = budget / per_step;
  return r < 1 ? 1 : (r > cap ? cap : r);
}

struct Variant {
  int bits, ug, lg, gg, ud, ld, gd, epl;
  bool operator<(const Variant& o) const {
    return std::tie(bits, ug, lg, gg, ud, ld, gd, epl) <
           std::tie(o.bits, o.ug, o.lg, o.gg, o.ud, o.ld, o.gd, o.epl);
  }
};

using FusedFn = void (*)(const FusedArgs, const RouteDev);
using XcdFn = void (*)(DecodeSync*, const int32_t*, const uint16_t*, const uint16_t*,
                       const float*, int, int, const FusedArgs, const RouteDev);

struct Entry {
  FusedFn fn;
  int sub_rows;  // down rows per wave item
};

struct XcdEntry {
  XcdFn fn;
  int sub_rows;
};

// Gate/up row steps per wave item and down row steps per down item (~16
// rows; 8 when a step already covers 8 rows).  Both split in two halves:
// even step counts (down: 1 when a step already covers 8 rows).
template <int UG, int GG>
constexpr int gateup_steps() {
  return (fused_r<UG, GG, true>(6) & ~1) < 2 ? 2 : (fused_r<UG, GG, true>(6) & ~1);
}
template <int UD, int LD, int GD>
constexpr int down_steps() {
  constexpr int RPW_D = 64 / LD;
  return RPW_D >= 8 ? 1 : ((fused_r<UD, GD, false>(16 / RPW_D) & ~1) < 2
                               ? 2 : (fused_r<UD, GD, false>(16 / RPW_D) & ~1));
}

template <int UG, int LG, int GG, int UD, int LD, int GD, int EPL>
Entry make_entry() {
  constexpr int RG = gateup_steps<UG, GG>(), RD = down_steps<UD, LD, GD>();
  return {&decode_fused_kernel<UG, LG, GG, RG, UD, LD, GD, RD, EPL>, RD * (64 / LD)};
}

template <int UG, int LG, int GG, int UD, int LD, int GD>
XcdEntry make_xcd_entry() {
  constexpr int RG = gateup_steps<UG, GG>(), RD = down_steps<UD, LD, GD>();
  return {&decode_xcd_kernel<UG, LG, GG, RG, UD, LD, GD, RD>, RD * (64 / LD)};
}

using ExpertsFn = void (*)(DecodeSync*, const int32_t*, const float*, int, int, const FusedArgs);
struct ExpertsEntry {
  ExpertsFn fn;
  int sub_rows;
};

template <int UG, int LG, int GG, int UD, int LD, int GD>
ExpertsEntry make_experts_entry() {
  constexpr int RG = gateup_steps<UG, GG>(), RD = down_steps<UD, LD, GD>();
  return {&experts_xcd_kernel<UG, LG, GG, RG, UD, LD, GD, RD>, RD * (64 / LD)};
}

// Supported (gate/up row shape, down row shape) pairs, from gateup_shape and
// pick_shape:
// 4-bit hidden 1024/inter 512, 4096/1536, 4096/2048, 7168/2048, 2048/512,
// 2048/768; 6-bit 1024/512, 4096/1536, 7168/2048, 2048/512; experts up to
// 512.  Other shapes use the three-launch path.
const std::map<Variant, Entry>& variants() {
  static const std::map<Variant, Entry> m = [] {
    std::map<Variant, Entry> v;
#define PMOE_FV(B, UG, LG, GG, UD, LD, GD, E) \
  v[{B, UG, LG, GG, UD, LD, GD, E}] = make_entry<UG, LG, GG, UD, LD, GD, E>();
#define PMOE_FV_E(B, UG, LG, GG, UD, LD, GD)                                    \
  PMOE_FV(B, UG, LG, GG, UD, LD, GD, 2) PMOE_FV(B, UG, LG, GG, UD, LD, GD, 4)   \
  PMOE_FV(B, UG, LG, GG, UD, LD, GD, 8)
    PMOE_FV_E(4, 16, 32, 1, 16, 16, 1)
    PMOE_FV_E(4, 32, 64, 2, 16, 64, 1)
    PMOE_FV_E(4, 16, 64, 2, 16, 16, 3)
    PMOE_FV_E(4, 16, 64, 2, 16, 64, 1)
    PMOE_FV_E(4, 16, 64, 1, 16, 16, 1)
    PMOE_FV_E(4, 16, 64, 1, 16, 8, 3)
    PMOE_FV_E(6, 48, 16, 1, 48, 8, 1)
    PMOE_FV_E(6, 48, 64, 1, 48, 32, 1)
    PMOE_FV_E(6, 48, 64, 2, 48, 32, 1)
    PMOE_FV_E(6, 48, 32, 1, 48, 8, 1)
#undef PMOE_FV_E
#undef PMOE_FV
    return v;
  }();
  return m;
}

// Expert-per-XCD variants (key epl = 0): the shapes of the grid-wide table
// except the 6-bit 48-lane-group down rows, whose gate/up + down prefetch
// registers exceed 256 VGPRs (those shapes keep the grid-wide launch).
const std::map<Variant, XcdEntry>& xcd_variants() {
  static const std::map<Variant, XcdEntry> m = [] {
    std::map<Variant, XcdEntry> v;
#define PMOE_XV(B, UG, LG, GG, UD, LD, GD) \
  v[{B, UG, LG, GG, UD, LD, GD, 0}] = make_xcd_entry<UG, LG, GG, UD, LD, GD>();
    PMOE_XV(4, 16, 32, 1, 16, 16, 1)
    PMOE_XV(4, 32, 64, 2, 16, 64, 1)
    PMOE_XV(4, 16, 64, 2, 16, 16, 3)
    PMOE_XV(4, 16, 64, 2, 16, 64, 1)
    PMOE_XV(4, 16, 64, 1, 16, 16, 1)
    PMOE_XV(4, 16, 64, 1, 16, 8, 3)
    PMOE_XV(6, 48, 16, 1, 48, 8, 1)
    PMOE_XV(6, 48, 32, 1, 48, 8, 1)
#undef PMOE_XV
    return v;
  }();
  return m;
}

// Given-ids expert-per-XCD variants: the same shapes.
const std::map<Variant, ExpertsEntry>& experts_variants() {
  static const std::map<Variant, ExpertsEntry> m = [] {
    std::map<Variant, ExpertsEntry> v;
#define PMOE_EV(B, UG, LG, GG, UD, LD, GD) \
  v[{B, UG, LG, GG, UD, LD, GD, 0}] = make_experts_entry<UG, LG, GG, UD, LD, GD>();
    PMOE_EV(4, 16, 32, 1, 16, 16, 1)
    PMOE_EV(4, 32, 64, 2, 16, 64, 1)
    PMOE_EV(4, 16, 64, 2, 16, 16, 3)
    PMOE_EV(4, 16, 64, 2, 16, 64, 1)
    PMOE_EV(4, 16, 64, 1, 16, 16, 1)
    PMOE_EV(4, 16, 64, 1, 16, 8, 3)
    PMOE_EV(6, 48, 16, 1, 48, 8, 1)
    PMOE_EV(6, 48, 32, 1, 48, 8, 1)
#undef PMOE_EV
    return v;
  }();
  return m;
}

bool xcd_enabled() {
  const char* v = getenv("PMOE_DECODE_XCD");
  return !(v && v[0] == '0');
}

// Blocks per launch: one per CU, provided the kernel fits one block per CU
// with this LDS size (checked once per device, kernel and size).
int fused_blocks(const void* fn, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, void*, size_t>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lk(mu);
  const auto key = std::make_tuple(dev, const_cast<void*>(fn), lds);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int cus = 0, nb = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, kFThreads, lds) != hipSuccess)
    nb = 0;
  const int blocks = nb >= 1 ? cus : 0;
  cache[key] = blocks;
  return blocks;
}

}  // namespace

extern "C" int pmoe_set_barrier_spin(uint64_t ticks) {
  pmoe::clear_error();
  g_spin_ticks = ticks ? ticks : kSpinTicks;
  return PMOE_OK;
}

extern "C" int pmoe_set_split_probe(int on) {
  pmoe::clear_error();
  g_split_probe = on ? 1u : 0u;
  return PMOE_OK;
}

#ifdef PMOE_FUSED_TRACE
extern "C" int pmoe_debug_trace(uint64_t* out, int n) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_trace), size_t(n) * sizeof(uint64_t)) == hipSuccess
             ? 0 : -2;
}
#endif

// The expert-per-XCD variant of a one-token layer and its grid, or nullptr.
static const XcdEntry* xcd_plan(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt,
                                int bits, bool gate_extra, int* blocks_out) {
  if (!(xcd_enabled() && rank1_route_ok(rt) && rt.k == kXcdCount && rt.kk == rt.k &&
        !gate_extra && dn.cols <= kXcdMaxInter && dn.rows_out <= kXcdMaxHidden &&
        rt.e + 128 <= kFThreads && rt.e <= int(kXcdLogitStride)))
    return nullptr;
  const Shape sg = gateup_shape(bits, gu, kXcdCount), sd = pick_shape(bits, dn.cols);
  const auto xt = xcd_variants().find({bits, sg.ub, sg.lpr, sg.gpl, sd.ub, sd.lpr, sd.gpl, 0});
  if (xt == xcd_variants().end()) return nullptr;
  const int blocks = fused_blocks(reinterpret_cast<const void*>(xt->second.fn), 0);
  const int per_xcd = blocks / kXcdCount;
  const int n_tiles = (dn.rows_out + xt->second.sub_rows - 1) / xt->second.sub_rows;
  if (!(blocks > 0 && blocks <= kDecodeMaxBlocks && blocks % kXcdCount == 0 &&
        (per_xcd & (per_xcd - 1)) == 0 && n_tiles <= kXcdMaxTiles &&
        rt.e <= kXcdLogitsPerWave * per_xcd * kFWaves))
    return nullptr;
  *blocks_out = blocks;
  return &xt->second;
}

bool decode_xcd_covers(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt, int bits,
                       bool gate_extra) {
  int blocks = 0;
  return xcd_plan(gu, dn, rt, bits, gate_extra, &blocks) != nullptr;
}

int decode_fused(const GemvArgs& gu, const GemvArgs& dn, const RouteDev& rt, int bits,
                 const uint16_t* x, const uint16_t* gate_w, const uint16_t* gate_extra,
                 const float* logit_bias, int32_t* inds_out, float* w_out, uint16_t* out,
                 DecodeSync* sync, hipStream_t st) {
  if (!sync || rt.n * rt.ld > kFMaxLogits) return kDecodeFusedDeclined;
  const int n_ids = rt.e + (rt.kk > rt.k ? 1 : 0);
  const int max_experts = rt.n * rt.kk < n_ids ? rt.n * rt.kk : n_ids;
  const Shape sg = gateup_shape(bits, gu, max_experts), sd = pick_shape(bits, dn.cols);
  const int epl = (rt.e + 63) / 64;
  const int epl_t = epl <= 2 ? 2 : (epl <= 4 ? 4 : (epl <= 8 ? 8 : 0));
  if (sg.lpr == 0 || sd.lpr == 0 || epl_t == 0) return kDecodeFusedDeclined;
  FusedArgs a{};
  a.x = x;
  a.gate_w = gate_w;
  a.gate_extra = gate_extra;
  a.logit_bias = logit_bias;
  a.logits = const_cast<float*>(rt.logits);
  a.gu = gu;
  a.dn = dn;
  a.out = out;
  a.inds_out = inds_out;
  a.w_out = w_out;
  a.sync = sync;
  a.spin = g_spin_ticks;
  a.split_probe = g_split_probe;
  // One token, top-8 softmax, no shared expert: the expert-per-XCD launch
  // when the grid splits into 8 groups of a power-of-two block count.
  int xblocks = 0;
  if (const XcdEntry* xe = xcd_plan(gu, dn, rt, bits, gate_extra != nullptr, &xblocks)) {
    a.n_blocks = xblocks;
    ProfScope prof_scope(K_DECODE_XCD, st);
    xe->fn<<<xblocks, kFThreads, 0, st>>>(a.sync, a.gu.table, a.x, a.gate_w, a.logit_bias,
                                          a.gu.cols, rt.e, a, rt);
    PMOE_LAUNCH_CHECK("decode_xcd_kernel");
    return PMOE_OK;
  }
  const auto& vs = variants();
  const auto it = vs.find({bits, sg.ub, sg.lpr, sg.gpl, sd.ub, sd.lpr, sd.gpl, epl_t});
  if (it == vs.end()) return kDecodeFusedDeclined;
  const Entry& en = it->second;
  // tile = down rows per block, a whole number of wave items
  int blocks = fused_blocks(reinterpret_cast<const void*>(en.fn), 0);
  if (blocks <= 0) return kDecodeFusedDeclined;
  const int per_block = (dn.rows_out + blocks - 1) / blocks;
  const int tile = (per_block + en.sub_rows - 1) / en.sub_rows * en.sub_rows;
  const size_t lds = size_t(rt.n) * rt.kk * tile * sizeof(float);
  if (lds > 64 * 1024) return kDecodeFusedDeclined;
  blocks = fused_blocks(reinterpret_cast<const void*>(en.fn), lds);
  if (blocks <= 0 || blocks > kDecodeMaxBlocks || blocks * tile < dn.rows_out)
    return kDecodeFusedDeclined;
  a.n_blocks = blocks;
  a.tile = tile;
  ProfScope prof_scope(K_DECODE_FUSED, st);
  en.fn<<<blocks, kFThreads, lds, st>>>(a, rt);
  PMOE_LAUNCH_CHECK("decode_fused_kernel");
  return PMOE_OK;
}

// The given-ids variant of a shape and its grid, or nullptr (nothing launched).
static const ExpertsEntry* experts_plan(const GemvArgs& gu, const GemvArgs& dn, int bits,
                                        int* blocks_out) {
  const char* v = getenv("PMOE_EXPERTS_XCD");
  if ((v && v[0] == '0') || !xcd_enabled()) return nullptr;
  if (dn.cols > kXcdMaxInter || dn.rows_out > kXcdMaxHidden) return nullptr;
  const Shape sg = gateup_shape(bits, gu, kXcdCount + 1), sd = pick_shape(bits, dn.cols);
  if (sg.lpr == 0 || sd.lpr == 0) return nullptr;
  const auto et = experts_variants().find({bits, sg.ub, sg.lpr, sg.gpl, sd.ub, sd.lpr, sd.gpl, 0});
  if (et == experts_variants().end()) return nullptr;
  const int blocks = fused_blocks(reinterpret_cast<const void*>(et->second.fn), 0);
  const int per_xcd = blocks / kXcdCount;
  const int n_tiles = (dn.rows_out + et->second.sub_rows - 1) / et->second.sub_rows;
  if (blocks <= 0 || blocks > kDecodeMaxBlocks || blocks % kXcdCount != 0 ||
      (per_xcd & (per_xcd - 1)) != 0 || n_tiles > kXcdMaxTiles)
    return nullptr;
  *blocks_out = blocks;
  return &et->second;
}

bool experts_xcd_covers(const GemvArgs& gu, const GemvArgs& dn, int bits, int) {
  int blocks = 0;
  return experts_plan(gu, dn, bits, &blocks) != nullptr;
}

int experts_xcd(const GemvArgs& gu, const GemvArgs& dn, int bits, int n_experts,
                const int32_t* ids, const float* wts, int shared_slot, uint16_t* out,
                DecodeSync* sync, hipStream_t st, bool round_y) {
  int blocks = 0;
  const ExpertsEntry* en = sync ? experts_plan(gu, dn, bits, &blocks) : nullptr;
  if (!en) return kDecodeFusedDeclined;
  FusedArgs a{};
  a.gu = gu;
  a.dn = dn;
  a.out = out;
  a.sync = sync;
  a.spin = g_spin_ticks;
  a.split_probe = g_split_probe;
  a.round_y = round_y ? 1u : 0u;
  a.n_blocks = blocks;
  ProfScope prof_scope(K_EXPERTS_XCD, st);
  en->fn<<<blocks, kFThreads, 0, st>>>(sync, ids, wts, n_experts, shared_slot, a);
  PMOE_LAUNCH_CHECK("experts_xcd_kernel");
  return PMOE_OK;
}

}  // namespace pmoe
