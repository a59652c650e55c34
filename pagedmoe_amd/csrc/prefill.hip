// Prefill expert GEMMs: expert-grouped, dequantize-in-registers, bf16 MFMA.
//
// Replaces the prefill branch of StreamedSwitchGLU._run (streaming.py:789-836:
// stable argsort of the flat ids, per-expert row groups, three
// mx.quantized_matmul per expert, unsort) with two kernels over the dispatch
// tiles (tile = up to kTileM rows of one expert, in dispatch order):
//
//   gateup_mfma_kernel: h[p, c] = silu(x_p . Wg[c]) * (x_p . Wu[c]) for the
//     tile's rows p (sorted positions) and 128 columns c of moe_intermediate;
//   down_mfma_kernel:   y[order[p], d] = h_p . Wd[d] for 256 columns d of hidden.
//
// Work split (256 threads = 4 waves): the tile's activation rows are staged
// through LDS one 64-wide quantization group at a time (double buffered) and
// shared by the 4 waves; each wave owns 64 weight rows (gate+up rows of 32
// columns, or 64 down rows), loads their packed words straight from HBM, and
// dequantizes them in registers into the MFMA B operand, so every weight
// byte is read and dequantized once per tile.  v_mfma_f32_32x32x16_bf16,
// fp32 accumulators.  The dequantized weight is bf16(fma(s, q, b)), the
// format's bf16 dequantization (quant.hip), like the bf16 tile loads of mlx's
// quantized GEMMs.
//
// K order.  For MFMA step s (16 of the group's 64 k) and lane half h, lane
// element i holds k = 32h + 8s + i: each lane's weight operand for a whole
// group is one contiguous run of packed bits, and the activation operand is
// read from LDS with the same mapping, so the dot product is unchanged.
#include "pmoe_internal.h"
#include "pmoe_kernels.h"

namespace pmoe {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileM = 128;          // rows per dispatch tile
constexpr int kMB = kTileM / 32;     // 32-row MFMA blocks per tile
constexpr int kLdsRow = 72;          // bf16 per staged row (64 + 8 pad: 144 B)
constexpr int kThreads = 256;
constexpr int kGuCols = 128;         // moe_intermediate columns per gate/up block
constexpr int kDnCols = 256;         // hidden columns per down block

struct PrefillArgs {
  const uint8_t* slab;
  int64_t expert_bytes;
  const int32_t* table;
  int n_experts;
  int shared_slot;
  const int32_t* order;
  const int32_t* counts;
  const int32_t* offsets;
  const int2* tiles;
  const int32_t* n_tiles;
  const uint16_t* act;   // gate/up: x [n, hidden]; down: h [rows, inter] in sorted order
  int kk;                // flat rows per token (gate/up activation gather)
  int cols;              // reduction length: hidden (gate/up) or inter (down)
  int64_t w0, s0, b0;    // component offsets of the first weight matrix
  int64_t w1, s1, b1;    // and of the second (up for gate/up; = first for down)
  int out_cols;          // inter (h) or hidden (y)
  void* out;
  int out_f32;
};

// Tile of this block: expert, first sorted position, row count, slot.
struct TileInfo {
  int e, p0, m, slot;
};

__device__ __forceinline__ TileInfo tile_info(const PrefillArgs& a, int t) {
  const int2 tl = a.tiles[t];
  TileInfo ti;
  ti.e = tl.x;
  const int cnt = a.counts[tl.x];
  ti.m = min(kTileM, cnt - tl.y);
  ti.p0 = a.offsets[tl.x] + tl.y;
  ti.slot = tl.x < a.n_experts ? a.table[tl.x] : a.shared_slot;
  return ti;
}

// ---------------------------------------------------------------- dequant

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }

// 8 consecutive 4-bit values of one word (low nibble first) -> bf16(s*q+b).
__device__ __forceinline__ bf16x8 deq8_4(uint32_t w, float s, float b) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // q0 q2 q4 q6
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // q1 q3 q5 q7
  bf16x8 r;
  r[0] = (__bf16)__builtin_fmaf(s, float(lo & 0xffu), b);
  r[1] = (__bf16)__builtin_fmaf(s, float(hi & 0xffu), b);
  r[2] = (__bf16)__builtin_fmaf(s, float((lo >> 8) & 0xffu), b);
  r[3] = (__bf16)__builtin_fmaf(s, float((hi >> 8) & 0xffu), b);
  r[4] = (__bf16)__builtin_fmaf(s, float((lo >> 16) & 0xffu), b);
  r[5] = (__bf16)__builtin_fmaf(s, float((hi >> 16) & 0xffu), b);
  r[6] = (__bf16)__builtin_fmaf(s, float(lo >> 24), b);
  r[7] = (__bf16)__builtin_fmaf(s, float(hi >> 24), b);
  return r;
}

// 6-bit field j of a little-endian bit stream held in words w[].
template <int J>
__device__ __forceinline__ uint32_t field6(const uint32_t* w) {
  constexpr int bit = 6 * J, wi = bit / 32, sh = bit % 32;
  if constexpr (sh <= 26)
    return (w[wi] >> sh) & 63u;
  else
    return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & 63u;
}

template <int S>
__device__ __forceinline__ bf16x8 deq8_6(const uint32_t* w, float s, float b) {
  bf16x8 r;
  r[0] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 0>(w)), b);
  r[1] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 1>(w)), b);
  r[2] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 2>(w)), b);
  r[3] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 3>(w)), b);
  r[4] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 4>(w)), b);
  r[5] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 5>(w)), b);
  r[6] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 6>(w)), b);
  r[7] = (__bf16)__builtin_fmaf(s, float(field6<8 * S + 7>(w)), b);
  return r;
}

// One lane's packed words of one group: values [32h, 32h + 32) of a row.
template <int BITS>
struct LaneWords {
  static constexpr int kWords = BITS;  // 32 values * BITS bits / 32
  uint32_t w[kWords];
};

template <int BITS>
__device__ __forceinline__ void load_words(LaneWords<BITS>& lw, const uint8_t* p) {
  if constexpr (BITS == 4) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    lw.w[0] = v[0];
    lw.w[1] = v[1];
    lw.w[2] = v[2];
    lw.w[3] = v[3];
  } else {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p) + j);
      lw.w[2 * j] = v[0];
      lw.w[2 * j + 1] = v[1];
    }
  }
}

template <int BITS>
__device__ __forceinline__ void dequant_group(const LaneWords<BITS>& lw, float s, float b,
                                              bf16x8 (&out)[4]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int st = 0; st < 4; ++st) out[st] = deq8_4(lw.w[st], s, b);
  } else {
    out[0] = deq8_6<0>(lw.w, s, b);
    out[1] = deq8_6<1>(lw.w, s, b);
    out[2] = deq8_6<2>(lw.w, s, b);
    out[3] = deq8_6<3>(lw.w, s, b);
  }
}

// ---------------------------------------------------------------- staging

// Rows of the tile's activations for group g -> registers (thread t holds
// row t/2, values [32*(t%2), +32)).  Rows past the tile are not loaded.
struct StageRegs {
  u32x4 v[4];
};

template <bool GATHER>
__device__ __forceinline__ void stage_load(const PrefillArgs& a, const TileInfo& ti,
                                           const uint16_t* row_src, int g, StageRegs& r) {
  const int row = threadIdx.x >> 1;
  if (row >= ti.m) return;
  const u32x4* src = reinterpret_cast<const u32x4*>(row_src + g * 64 + (threadIdx.x & 1) * 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) r.v[j] = src[j];
}

__device__ __forceinline__ void stage_store(uint16_t* lds, const StageRegs& r, int m) {
  const int row = threadIdx.x >> 1;
  if (row >= m) return;
  u32x4* dst = reinterpret_cast<u32x4*>(lds + row * kLdsRow + (threadIdx.x & 1) * 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) dst[j] = r.v[j];
}

// ---------------------------------------------------------------- main loop

// acc0/acc1[mb] += A_tile(mb) . B0/B1 over the whole reduction.  B0 is weight
// row ptr0 (+ scales/biases s0p/b0p), B1 weight row ptr1.
template <int BITS, bool GATHER>
__device__ __forceinline__ void gemm_tile(const PrefillArgs& a, const TileInfo& ti,
                                          const uint16_t* row_src, const uint8_t* wp0,
                                          const uint16_t* sp0, const uint16_t* bp0,
                                          const uint8_t* wp1, const uint16_t* sp1,
                                          const uint16_t* bp1, uint16_t* lds,
                                          f32x16 (&acc0)[kMB], f32x16 (&acc1)[kMB]) {
  constexpr int kGroupBytes = 64 * BITS / 8;
  const int lane = threadIdx.x & 63;
  const int m = lane & 31;
  const int h = lane >> 5;
  const int n_groups = a.cols / 64;
  const int nmb = (ti.m + 31) >> 5;
  const uint8_t* wl0 = wp0 + h * (kGroupBytes / 2);
  const uint8_t* wl1 = wp1 + h * (kGroupBytes / 2);

#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    acc0[mb] = f32x16{};
    acc1[mb] = f32x16{};
  }

  StageRegs sr;
  stage_load<GATHER>(a, ti, row_src, 0, sr);
  LaneWords<BITS> cw0, cw1;
  load_words<BITS>(cw0, wl0);
  load_words<BITS>(cw1, wl1);
  uint32_t cs0 = sp0[0], cb0 = bp0[0], cs1 = sp1[0], cb1 = bp1[0];
  stage_store(lds, sr, ti.m);
  __syncthreads();

  for (int g = 0; g < n_groups; ++g) {
    const bool more = g + 1 < n_groups;
    LaneWords<BITS> nw0, nw1;
    uint32_t ns0 = 0, nb0 = 0, ns1 = 0, nb1 = 0;
    if (more) {
      stage_load<GATHER>(a, ti, row_src, g + 1, sr);
      load_words<BITS>(nw0, wl0 + size_t(g + 1) * kGroupBytes);
      load_words<BITS>(nw1, wl1 + size_t(g + 1) * kGroupBytes);
      ns0 = sp0[g + 1];
      nb0 = bp0[g + 1];
      ns1 = sp1[g + 1];
      nb1 = bp1[g + 1];
    }
    bf16x8 b0[4], b1[4];
    dequant_group<BITS>(cw0, bf_lo(cs0), bf_lo(cb0), b0);
    dequant_group<BITS>(cw1, bf_lo(cs1), bf_lo(cb1), b1);
    const uint16_t* xs = lds + (g & 1) * (kTileM * kLdsRow);
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
      if (mb < nmb) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const bf16x8 av =
              *reinterpret_cast<const bf16x8*>(xs + (mb * 32 + m) * kLdsRow + 32 * h + 8 * st);
          acc0[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b0[st], acc0[mb], 0, 0, 0);
          acc1[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b1[st], acc1[mb], 0, 0, 0);
        }
      }
    }
    if (more) {
      stage_store(lds + ((g + 1) & 1) * (kTileM * kLdsRow), sr, ti.m);
      cw0 = nw0;
      cw1 = nw1;
      cs0 = ns0;
      cb0 = nb0;
      cs1 = ns1;
      cb1 = nb1;
    }
    __syncthreads();
  }
}

// Row of accumulator register r of a 32x32 block for lane half h.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// ---------------------------------------------------------------- kernels

template <int BITS>
__global__ __launch_bounds__(kThreads) void gateup_mfma_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kTileM * kLdsRow];
  if (int(blockIdx.y) >= *a.n_tiles) return;
  const TileInfo ti = tile_info(a, blockIdx.y);
  if (ti.slot < 0) return;  // the down kernel writes this tile's zero rows
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = blockIdx.x * kGuCols + wave * 32 + (lane & 31);
  const uint8_t* base = a.slab + size_t(ti.slot) * size_t(a.expert_bytes);
  const size_t row_bytes = size_t(a.cols) * BITS / 8;
  const int groups = a.cols / 64;
  // activation row of this thread's staging row (token of the flat row)
  const int srow = threadIdx.x >> 1;
  const uint16_t* row_src = a.act;
  if (srow < ti.m) row_src = a.act + size_t(a.order[ti.p0 + srow] / a.kk) * a.cols;
  f32x16 accg[kMB], accu[kMB];
  gemm_tile<BITS, true>(
      a, ti, row_src, base + a.w0 + col * row_bytes,
      reinterpret_cast<const uint16_t*>(base + a.s0) + size_t(col) * groups,
      reinterpret_cast<const uint16_t*>(base + a.b0) + size_t(col) * groups,
      base + a.w1 + col * row_bytes,
      reinterpret_cast<const uint16_t*>(base + a.s1) + size_t(col) * groups,
      reinterpret_cast<const uint16_t*>(base + a.b1) + size_t(col) * groups, lds, accg, accu);
  uint16_t* hout = static_cast<uint16_t*>(a.out);
  const int h = lane >> 5;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = mb * 32 + acc_row(r, h);
      if (row < ti.m) {
        const float v = silu_fast(accg[mb][r]) * accu[mb][r];
        hout[size_t(ti.p0 + row) * a.out_cols + col] = f2bf(v);
      }
    }
  }
}

template <int BITS>
__global__ __launch_bounds__(kThreads) void down_mfma_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kTileM * kLdsRow];
  if (int(blockIdx.y) >= *a.n_tiles) return;
  const TileInfo ti = tile_info(a, blockIdx.y);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col0 = blockIdx.x * kDnCols + wave * 64 + (lane & 31);
  const int col1 = col0 + 32;
  const int h = lane >> 5;
  if (ti.slot < 0) {  // not resident: exact zero rows (streaming.py:715-719)
    for (int row = h; row < ti.m; row += 2) {
      const size_t o = size_t(a.order[ti.p0 + row]) * a.out_cols;
      if (a.out_f32) {
        static_cast<float*>(a.out)[o + col0] = 0.0f;
        static_cast<float*>(a.out)[o + col1] = 0.0f;
      } else {
        static_cast<uint16_t*>(a.out)[o + col0] = 0;
        static_cast<uint16_t*>(a.out)[o + col1] = 0;
      }
    }
    return;
  }
  const uint8_t* base = a.slab + size_t(ti.slot) * size_t(a.expert_bytes);
  const size_t row_bytes = size_t(a.cols) * BITS / 8;
  const int groups = a.cols / 64;
  const int srow = threadIdx.x >> 1;
  const uint16_t* row_src = a.act + size_t(ti.p0 + (srow < ti.m ? srow : 0)) * a.cols;
  const uint16_t* sp = reinterpret_cast<const uint16_t*>(base + a.s0);
  const uint16_t* bp = reinterpret_cast<const uint16_t*>(base + a.b0);
  f32x16 acc0[kMB], acc1[kMB];
  gemm_tile<BITS, false>(a, ti, row_src, base + a.w0 + col0 * row_bytes,
                         sp + size_t(col0) * groups, bp + size_t(col0) * groups,
                         base + a.w0 + col1 * row_bytes, sp + size_t(col1) * groups,
                         bp + size_t(col1) * groups, lds, acc0, acc1);
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = mb * 32 + acc_row(r, h);
      if (row < ti.m) {
        const size_t o = size_t(a.order[ti.p0 + row]) * a.out_cols;
        if (a.out_f32) {
          static_cast<float*>(a.out)[o + col0] = acc0[mb][r];
          static_cast<float*>(a.out)[o + col1] = acc1[mb][r];
        } else {
          static_cast<uint16_t*>(a.out)[o + col0] = f2bf(acc0[mb][r]);
          static_cast<uint16_t*>(a.out)[o + col1] = f2bf(acc1[mb][r]);
        }
      }
    }
  }
}

}  // namespace

int prefill_tile_m() { return kTileM; }

// The MFMA path pays off once experts see tens of rows; below that the
// weight-streaming GEMV (decode.hip) is as fast and needs no tile list.
bool prefill_wanted(const pmoe_geom* g, int n, int kk, int n_ids) {
  const long rows = long(n) * kk;
  if (g->inter % kGuCols || g->hidden % kDnCols) return false;
  return rows >= 1024 && rows >= 16L * n_ids;
}

int prefill_experts(const pmoe_geom* g, const uint8_t* slab, const int32_t* table, int n_experts,
                    int shared_slot, const uint16_t* x, int n, int kk, const int32_t* order,
                    const int32_t* counts, const int32_t* offsets, const int2* tiles,
                    const int32_t* n_tiles, int max_tiles, uint16_t* h, void* y, int y_f32,
                    hipStream_t st) {
  (void)n;
  PMOE_REQUIRE(g->inter % kGuCols == 0 && g->hidden % kDnCols == 0,
               "prefill: inter must be a multiple of 128 and hidden of 256");
  PMOE_REQUIRE(max_tiles > 0 && max_tiles <= 65535, "prefill: tile count out of range");
  PrefillArgs a{};
  a.slab = slab;
  a.expert_bytes = g->expert_bytes;
  a.table = table;
  a.n_experts = n_experts;
  a.shared_slot = shared_slot;
  a.order = order;
  a.counts = counts;
  a.offsets = offsets;
  a.tiles = tiles;
  a.n_tiles = n_tiles;
  // gate + up -> h (sorted rows)
  a.act = x;
  a.kk = kk;
  a.cols = g->hidden;
  a.w0 = g->off[PMOE_GATE_W];
  a.s0 = g->off[PMOE_GATE_S];
  a.b0 = g->off[PMOE_GATE_B];
  a.w1 = g->off[PMOE_UP_W];
  a.s1 = g->off[PMOE_UP_S];
  a.b1 = g->off[PMOE_UP_B];
  a.out_cols = g->inter;
  a.out = h;
  a.out_f32 = 0;
  {
    dim3 grid(g->inter / kGuCols, max_tiles);
    ProfScope prof_scope(K_PREFILL_GATEUP, st);
    if (g->bits == 4)
      gateup_mfma_kernel<4><<<grid, kThreads, 0, st>>>(a);
    else
      gateup_mfma_kernel<6><<<grid, kThreads, 0, st>>>(a);
    PMOE_LAUNCH_CHECK("gateup_mfma_kernel");
  }
  // down -> y (flat rows)
  a.act = h;
  a.kk = 1;
  a.cols = g->inter;
  a.w0 = a.w1 = g->off[PMOE_DOWN_W];
  a.s0 = a.s1 = g->off[PMOE_DOWN_S];
  a.b0 = a.b1 = g->off[PMOE_DOWN_B];
  a.out_cols = g->hidden;
  a.out = y;
  a.out_f32 = y_f32;
  {
    dim3 grid(g->hidden / kDnCols, max_tiles);
    ProfScope prof_scope(K_PREFILL_DOWN, st);
    if (g->bits == 4)
      down_mfma_kernel<4><<<grid, kThreads, 0, st>>>(a);
    else
      down_mfma_kernel<6><<<grid, kThreads, 0, st>>>(a);
    PMOE_LAUNCH_CHECK("down_mfma_kernel");
  }
  return PMOE_OK;
}

}  // namespace pmoe
