// Token -> expert dispatch: histogram, exclusive scan, stable scatter.
//
// Replaces the reference's host-side dispatch: order = np.argsort(flat,
// kind="stable"), rows = order // K, per-expert searchsorted
// (streaming.py:789-808) and the unsort inv[order] = arange (:833-836).
// Integer work, HBM/latency bound; no float anywhere, so every output is
// bit-exact.
//
// Stability: the position of flat row r inside expert e's segment is the
// number of earlier rows with the same expert.  Rows are cut into blocks of
// kChunk; a row's rank inside its block comes from a broadcast LDS scan of the
// earlier rows of the block, and the block's base per expert from an
// exclusive scan over blocks (block-major within each expert).
#include "pmoe_internal.h"
#include "pmoe_kernels.h"

namespace pmoe {

namespace {

constexpr int kChunk = 256;        // rows per block in the multi-block path
constexpr int kSmallRows = 1024;   // single-kernel path up to this many rows
constexpr int kMaxExperts = 1024;

// Source of flat row ids: row r = n*kk + c reads inds[n*k_routed + c] for
// c < k_routed (valid in [0, n_routed)) and the shared pseudo-id n_routed for
// the extra column.  Returns -1 for an id out of range.
struct IdSrc {
  const int32_t* inds;
  int k_routed, kk, n_routed;
};

__device__ __forceinline__ int load_id(const IdSrc& src, int r) {
  const int n = r / src.kk;
  const int c = r - n * src.kk;
  if (c >= src.k_routed) return src.n_routed;
  const int e = src.inds[size_t(n) * src.k_routed + c];
  return (e >= 0 && e < src.n_routed) ? e : -1;
}

// Exclusive scans of three ints per thread over a block of NT threads, side
// by side (their shuffles overlap and they share the barriers).  s_tmp holds
// 3 * NT/64 ints.  v[i] becomes the exclusive prefix of v[i]; total[i] gets
// the sum.
template <int NT>
__device__ __forceinline__ void block_excl_scan3(int (&v)[3], int* s_tmp, int (&total)[3]) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int incl[3] = {v[0], v[1], v[2]};
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int o[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) o[i] = __shfl_up(incl[i], off, kWave);
#pragma unroll
    for (int i = 0; i < 3; ++i)
      if (lane >= off) incl[i] += o[i];
  }
  if (lane == 63)
#pragma unroll
    for (int i = 0; i < 3; ++i) s_tmp[i * NW + wave] = incl[i];
  __syncthreads();
  if (wave == 0) {
    int wi[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) wi[i] = lane < NW ? s_tmp[i * NW + lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      int o[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) o[i] = __shfl_up(wi[i], off, kWave);
#pragma unroll
      for (int i = 0; i < 3; ++i)
        if (lane >= off) wi[i] += o[i];
    }
    if (lane < NW)
#pragma unroll
      for (int i = 0; i < 3; ++i) s_tmp[i * NW + lane] = wi[i];  // inclusive wave totals
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int base = wave > 0 ? s_tmp[i * NW + wave - 1] : 0;
    total[i] = s_tmp[i * NW + NW - 1];
    v[i] = base + incl[i] - v[i];
  }
  __syncthreads();
}

// The prefill GEMMs' tile list (when tile_m > 0): tile t of expert e with
// c rows is {slot of e, t * tile_m, c, offset of e}, everything a GEMM block
// needs to find its rows and weights in one load.  Slots come from the slot
// table (routed ids below n_routed) or are the shared expert's.
struct TileSink {
  int4* tiles;
  int32_t* n_tiles;
  int tile_m;
  const int32_t* table;
  int n_routed, shared_slot;
};

// Per-expert totals -> counts, offsets, active list, n_active and the tile
// list.  Run by a block of 1024 threads; cnt[] is in LDS, one entry per
// expert.
__device__ void finish_scan(const int* cnt, int n_experts, int32_t* counts, int32_t* offsets,
                            int32_t* active, int32_t* n_active, const TileSink& ts, int* s_off,
                            int* s_tmp) {
  const int tile_m = ts.tile_m;
  const int e = threadIdx.x;
  const int c = e < n_experts ? cnt[e] : 0;
  const int nt = tile_m > 0 ? (c + tile_m - 1) / tile_m : 0;
  int sc[3] = {c, c > 0 ? 1 : 0, nt};  // rows, active experts, tiles
  int tot[3];
  block_excl_scan3<1024>(sc, s_tmp, tot);
  const int off = sc[0], act = sc[1], toff = sc[2];
  const int total = tot[0], act_total = tot[1], tiles_total = tot[2];
  if (e < n_experts) {
    s_off[e] = off;
    counts[e] = c;
    offsets[e] = off;
    if (c > 0) active[act] = e;
    if (nt > 0) {
      const int slot = e < ts.n_routed ? ts.table[e] : ts.shared_slot;
      for (int t = 0; t < nt; ++t) ts.tiles[toff + t] = make_int4(slot, t * tile_m, c, off);
    }
  }
  if (e == 0) {
    offsets[n_experts] = total;
    *n_active = act_total;
    if (tile_m > 0) *ts.n_tiles = tiles_total;
  }
  __syncthreads();
}

// Whole dispatch in one block (rows <= kSmallRows).
__global__ __launch_bounds__(1024) void dispatch_small_kernel(
    const IdSrc src, int rows, int n_experts, int32_t* __restrict__ order,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ inv,
    int32_t* __restrict__ active, int32_t* __restrict__ n_active, const TileSink ts) {
  __shared__ int s_e[kSmallRows];
  __shared__ int s_cnt[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_tmp[48];
  const int tid = threadIdx.x;
  for (int e = tid; e < n_experts; e += 1024) s_cnt[e] = 0;
  int my_e = -1;
  if (tid < rows) {
    my_e = load_id(src, tid);
    s_e[tid] = my_e;
  }
  __syncthreads();
  int rank = 0;
  if (my_e >= 0) {
    atomicAdd(&s_cnt[my_e], 1);
    for (int j = 0; j < tid; ++j) rank += (s_e[j] == my_e);
  }
  __syncthreads();
  finish_scan(s_cnt, n_experts, counts, offsets, active, n_active, ts, s_off, s_tmp);
  if (my_e >= 0) {
    const int pos = s_off[my_e] + rank;
    order[pos] = tid;
    inv[tid] = pos;
  } else if (tid < rows) {
    inv[tid] = -1;
  }
}

// Multi-block path, phase 1: per-block histogram and in-block ranks.
__global__ __launch_bounds__(kChunk) void dispatch_count_kernel(
    const IdSrc src, int rows, int n_experts, int32_t* __restrict__ hist,
    int32_t* __restrict__ rank_out) {
  __shared__ int s_e[kChunk];
  __shared__ int s_h[kMaxExperts];
  const int tid = threadIdx.x;
  const int row = blockIdx.x * kChunk + tid;
  for (int e = tid; e < n_experts; e += kChunk) s_h[e] = 0;
  int my_e = -1;
  if (row < rows) my_e = load_id(src, row);
  s_e[tid] = my_e;
  __syncthreads();
  if (my_e >= 0) {
    atomicAdd(&s_h[my_e], 1);
    int rank = 0;
    for (int j = 0; j < tid; ++j) rank += (s_e[j] == my_e);
    rank_out[row] = rank;
  }
  __syncthreads();
  for (int e = tid; e < n_experts; e += kChunk) hist[size_t(blockIdx.x) * n_experts + e] = s_h[e];
}

// Phase 2 (one block): turn hist[b][e] into each block's base position per
// expert and produce counts/offsets/active/tiles.  Thread e walks column e of
// hist; its first kKeep entries are loaded in one round (all in flight) and
// kept in registers for the second pass, so up to kKeep blocks (16,384 rows)
// cost one round of loads instead of two passes of dependent rounds.
__global__ __launch_bounds__(1024) void dispatch_scan_kernel(
    int32_t* __restrict__ hist, int n_blocks, int n_experts, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ active, int32_t* __restrict__ n_active,
    const TileSink ts) {
  __shared__ int s_cnt[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_tmp[48];
  constexpr int kKeep = 64;   // block histograms held in registers
  constexpr int kBatch = 16;  // further block histograms read per round, all in flight
  const int e = threadIdx.x;
  int hk[kKeep];
  if (e < n_experts) {
    // clamped index: straight-line loads, no branch per entry (n_blocks >= 1),
    // every load issued before the first is used
#pragma unroll
    for (int j = 0; j < kKeep; ++j)
      hk[j] = hist[size_t(j < n_blocks ? j : n_blocks - 1) * n_experts + e];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kKeep; ++j) hk[j] = j < n_blocks ? hk[j] : 0;
    int run = 0;
#pragma unroll
    for (int j = 0; j < kKeep; ++j) run += hk[j];
    for (int b0 = kKeep; b0 < n_blocks; b0 += kBatch) {
      int h[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        h[j] = b0 + j < n_blocks ? hist[size_t(b0 + j) * n_experts + e] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) run += h[j];
    }
    s_cnt[e] = run;
  }
  __syncthreads();
  finish_scan(s_cnt, n_experts, counts, offsets, active, n_active, ts, s_off, s_tmp);
  if (e < n_experts) {
    // each block's base position per expert: expert offset + earlier blocks
    int run = s_off[e];
#pragma unroll
    for (int j = 0; j < kKeep; ++j) {
      if (j < n_blocks) hist[size_t(j) * n_experts + e] = run;
      run += hk[j];
    }
    for (int b0 = kKeep; b0 < n_blocks; b0 += kBatch) {
      int h[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        h[j] = b0 + j < n_blocks ? hist[size_t(b0 + j) * n_experts + e] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (b0 + j < n_blocks) hist[size_t(b0 + j) * n_experts + e] = run;
        run += h[j];
      }
    }
  }
}

// Phase 3: scatter rows to their positions.
__global__ __launch_bounds__(kChunk) void dispatch_scatter_kernel(
    const IdSrc src, int rows, int n_experts, const int32_t* __restrict__ hist,
    const int32_t* __restrict__ rank, int32_t* __restrict__ order, int32_t* __restrict__ inv) {
  const int row = blockIdx.x * kChunk + threadIdx.x;
  if (row >= rows) return;
  const int e = load_id(src, row);
  if (e < 0) {
    inv[row] = -1;
    return;
  }
  const int pos = hist[size_t(blockIdx.x) * n_experts + e] + rank[row];
  order[pos] = row;
  inv[row] = pos;
}

}  // namespace

size_t dispatch_workspace(int rows, int n_experts) {
  if (rows <= kSmallRows) return 256;
  const size_t blocks = (rows + kChunk - 1) / kChunk;
  return ((blocks * n_experts + rows) * sizeof(int32_t) + 255) / 256 * 256;
}

// Internal entry: also builds the prefill tile list when tile_m > 0 (slots
// from table, the shared pseudo-id's from shared_slot).  Ids outside their
// range are dropped: counted nowhere, inv = -1.
int dispatch_ext(const int32_t* inds, int rows, int k_routed, int kk, int n_ids, int32_t* order,
                 int32_t* counts, int32_t* offsets, int32_t* inv, int32_t* active,
                 int32_t* n_active, int tile_m, int4* tiles, int32_t* n_tiles,
                 const int32_t* table, int shared_slot, void* ws, size_t ws_bytes,
                 hipStream_t st) {
  PMOE_REQUIRE(n_ids > 0 && n_ids <= kMaxExperts, "dispatch: experts must be 1..1024");
  PMOE_REQUIRE(rows >= 0, "dispatch: negative rows");
  PMOE_REQUIRE(k_routed >= 1 && kk >= k_routed && kk <= k_routed + 1, "dispatch: bad columns");
  PMOE_REQUIRE(rows % kk == 0, "dispatch: rows must be a multiple of the columns");
  const IdSrc src{inds, k_routed, kk, kk > k_routed ? n_ids - 1 : n_ids};
  PMOE_REQUIRE(tile_m == 0 || (tiles && n_tiles && table), "dispatch: tile list needs the slot table");
  const TileSink ts{tiles, n_tiles, tile_m, table, src.n_routed, shared_slot};
  ProfScope prof_scope(K_DISPATCH, st);
  if (rows <= kSmallRows) {
    dispatch_small_kernel<<<1, 1024, 0, st>>>(src, rows, n_ids, order, counts, offsets, inv,
                                              active, n_active, ts);
    PMOE_LAUNCH_CHECK("dispatch_small_kernel");
    return PMOE_OK;
  }
  PMOE_REQUIRE(ws != nullptr && ws_bytes >= dispatch_workspace(rows, n_ids),
               "dispatch: workspace too small");
  const int blocks = (rows + kChunk - 1) / kChunk;
  int32_t* hist = static_cast<int32_t*>(ws);
  int32_t* rank = hist + size_t(blocks) * n_ids;
  dispatch_count_kernel<<<blocks, kChunk, 0, st>>>(src, rows, n_ids, hist, rank);
  PMOE_LAUNCH_CHECK("dispatch_count_kernel");
  dispatch_scan_kernel<<<1, 1024, 0, st>>>(hist, blocks, n_ids, counts, offsets, active,
                                           n_active, ts);
  PMOE_LAUNCH_CHECK("dispatch_scan_kernel");
  dispatch_scatter_kernel<<<blocks, kChunk, 0, st>>>(src, rows, n_ids, hist, rank, order, inv);
  PMOE_LAUNCH_CHECK("dispatch_scatter_kernel");
  return PMOE_OK;
}

}  // namespace pmoe

extern "C" size_t pmoe_dispatch_workspace(int rows, int n_experts) {
  return pmoe::dispatch_workspace(rows, n_experts);
}

extern "C" int pmoe_dispatch(const int32_t* inds, int rows, int n_experts, int32_t* order,
                             int32_t* counts, int32_t* offsets, int32_t* inv, int32_t* active,
                             int32_t* n_active, void* ws, size_t ws_bytes, void* stream) {
  pmoe::clear_error();
  return pmoe::dispatch_ext(inds, rows, 1, 1, n_experts, order, counts, offsets, inv, active,
                            n_active, 0, nullptr, nullptr, nullptr, -1, ws, ws_bytes,
                            static_cast<hipStream_t>(stream));
}
