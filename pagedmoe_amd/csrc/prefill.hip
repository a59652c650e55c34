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
  r[0] = (__bf16)__builtin_fmaf(s, float(uint8_t(lo)), b);
  r[1] = (__bf16)__builtin_fmaf(s, float(uint8_t(hi)), b);
  r[2] = (__bf16)__builtin_fmaf(s, float(uint8_t(lo >> 8)), b);
  r[3] = (__bf16)__builtin_fmaf(s, float(uint8_t(hi >> 8)), b);
  r[4] = (__bf16)__builtin_fmaf(s, float(uint8_t(lo >> 16)), b);
  r[5] = (__bf16)__builtin_fmaf(s, float(uint8_t(hi >> 16)), b);
  r[6] = (__bf16)__builtin_fmaf(s, float(lo >> 24), b);
  r[7] = (__bf16)__builtin_fmaf(s, float(hi >> 24), b);
  return r;
}

// Byte n of v as float (v_cvt_f32_ubyteN).  Written as asm so the compiler
// keeps the shared nibble masks instead of re-extracting each field.
template <int N>
__device__ __forceinline__ float ubyte_f(uint32_t v) {
  float f;
  if constexpr (N == 0)
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (N == 1)
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (N == 2)
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(v));
  else
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(v));
  return f;
}

// Half HF (values 4*HF .. 4*HF+3) of one 4-bit word, lo = w & 0x0F0F0F0F
// (even values), hi = (w >> 4) & 0x0F0F0F0F (odd values), into o[4HF..].
template <int HF>
__device__ __forceinline__ void deq4_half(uint32_t lo, uint32_t hi, float s, float b,
                                          bf16x8& o) {
  o[4 * HF + 0] = (__bf16)__builtin_fmaf(s, ubyte_f<2 * HF>(lo), b);
  o[4 * HF + 1] = (__bf16)__builtin_fmaf(s, ubyte_f<2 * HF>(hi), b);
  o[4 * HF + 2] = (__bf16)__builtin_fmaf(s, ubyte_f<2 * HF + 1>(lo), b);
  o[4 * HF + 3] = (__bf16)__builtin_fmaf(s, ubyte_f<2 * HF + 1>(hi), b);
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

// Plain (cached) loads: a lane reads 16 or 24 bytes of a row per group, so
// one 128-byte line serves several consecutive groups and must stay in L2.
template <int BITS>
__device__ __forceinline__ void load_words(LaneWords<BITS>& lw, const uint8_t* p) {
  if constexpr (BITS == 4) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    lw.w[0] = v[0];
    lw.w[1] = v[1];
    lw.w[2] = v[2];
    lw.w[3] = v[3];
  } else {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const u32x2 v = reinterpret_cast<const u32x2*>(p)[j];
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

// One group (64 values) of the tile's activation rows -> registers.
// Piece p = 256*j + t (j < kMB) of the 16-byte pieces is row p / 8,
// chunk p % 8, so each load instruction covers whole 128-byte row segments.
// Rows past the tile re-load the tile's last row: every load stays in bounds
// and the code has no branch; the MFMA rows they feed are never stored.
struct StageRows {
  const uint16_t* base;
  uint32_t off[kMB];  // element offset of each staged row
};

struct StageRegs {
  u32x4 v[kMB];
};

// Only the first NMB 32-row blocks are staged.
template <int NMB>
__device__ __forceinline__ void stage_load(const StageRows& sr, int g, StageRegs& x) {
  const int c = threadIdx.x & 7;
#pragma unroll
  for (int j = 0; j < NMB; ++j)
    x.v[j] = *reinterpret_cast<const u32x4*>(sr.base + sr.off[j] + g * 64 + c * 8);
}

template <int NMB>
__device__ __forceinline__ void stage_store(uint16_t* lds, const StageRegs& x) {
  const int c = threadIdx.x & 7;
  const int r0 = threadIdx.x >> 3;
#pragma unroll
  for (int j = 0; j < NMB; ++j)
    *reinterpret_cast<u32x4*>(lds + (32 * j + r0) * kLdsRow + c * 8) = x.v[j];
}

// ---------------------------------------------------------------- main loop

// Per-lane weight rows: two rows (gate+up of one column, or two down rows),
// with their scale/bias rows (bf16, one per group, read 8 groups at a time).
struct LaneRows {
  const uint8_t* w0;
  const uint8_t* w1;
  const u32x4* s0;
  const u32x4* b0;
  const u32x4* s1;
  const u32x4* b1;
};

template <int BITS>
struct WSet {
  LaneWords<BITS> w0, w1;
};

// Scales and biases of 8 consecutive groups for both rows.
struct SBlk {
  u32x4 s0, b0, s1, b1;
};

template <int BITS>
__device__ __forceinline__ void load_wset(WSet<BITS>& ws, const LaneRows& lr, int g) {
  constexpr int kGroupBytes = 64 * BITS / 8;
  load_words<BITS>(ws.w0, lr.w0 + size_t(g) * kGroupBytes);
  load_words<BITS>(ws.w1, lr.w1 + size_t(g) * kGroupBytes);
}

__device__ __forceinline__ void load_sblk(SBlk& sb, const LaneRows& lr, int blk) {
  sb.s0 = lr.s0[blk];
  sb.b0 = lr.b0[blk];
  sb.s1 = lr.s1[blk];
  sb.b1 = lr.b1[blk];
}

// bf16 entry i (0..7) of 8 packed in a u32x4, as float.
__device__ __forceinline__ float bf_at(const u32x4& v, int i) {
  const uint32_t w = v[i >> 1];
  return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
}

// Dequant job jb (0..15) of a weight set: half jb & 1 (4 values) of MFMA
// step (jb >> 1) & 3 of row 0 (jb < 8) or row 1, with the group's
// scale/bias at entry i of sb.  Sixteen small jobs per group let the
// dequant spread evenly between the MFMAs.
template <int BITS>
__device__ __forceinline__ void dequant_job(const WSet<BITS>& ws, const SBlk& sb, int i, int jb,
                                            bf16x8 (&o0)[4], bf16x8 (&o1)[4]) {
  const bool r1 = jb >= 8;
  const int st = (jb >> 1) & 3;
  const LaneWords<BITS>& lw = r1 ? ws.w1 : ws.w0;
  const float s = bf_at(r1 ? sb.s1 : sb.s0, i);
  const float b = bf_at(r1 ? sb.b1 : sb.b0, i);
  bf16x8& o = r1 ? o1[st] : o0[st];
  if constexpr (BITS == 4) {
    const uint32_t w = lw.w[st];
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    if (jb & 1)
      deq4_half<1>(lo, hi, s, b, o);
    else
      deq4_half<0>(lo, hi, s, b, o);
  } else {
    bf16x8 t;
    switch (st) {
      case 0: t = deq8_6<0>(lw.w, s, b); break;
      case 1: t = deq8_6<1>(lw.w, s, b); break;
      case 2: t = deq8_6<2>(lw.w, s, b); break;
      default: t = deq8_6<3>(lw.w, s, b); break;
    }
    if (jb & 1) {
      o[4] = t[4]; o[5] = t[5]; o[6] = t[6]; o[7] = t[7];
    } else {
      o[0] = t[0]; o[1] = t[1]; o[2] = t[2]; o[3] = t[3];
    }
  }
}

// acc0/acc1[mb] = A_tile(mb) . B0/B1 over the whole reduction, for the
// tile's first NMB 32-row blocks.  Software pipeline (per quantization group
// j): weights of group j+3 and activations of group j+2 are in flight, group
// j+1's weights are dequantized while group j's MFMAs run, and group j+1's
// activations go to the other LDS buffer.  Scales/biases arrive 8 groups at
// a time, one block ahead.  The loop is unrolled by 8 so the register rings
// are indexed statically; loads past the end clamp to the last group (their
// data is unused).  n_groups is a multiple of 8.
template <int BITS, int NMB>
__device__ __forceinline__ void gemm_tile(int n_groups, const StageRows& rows,
                                          const LaneRows& lr, uint16_t* lds,
                                          f32x16 (&acc0)[kMB], f32x16 (&acc1)[kMB]) {
  const int lane = threadIdx.x & 63;
  const int m = lane & 31;
  const int h = lane >> 5;
  const int last = n_groups - 1;
  const int last_blk = (n_groups >> 3) - 1;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    acc0[mb] = f32x16{};
    acc1[mb] = f32x16{};
  }
  WSet<BITS> W[4];
  StageRegs X[NMB > 4 ? 1 : 2];
  SBlk S[2];
  bf16x8 B0[2][4], B1[2][4];
  load_sblk(S[0], lr, 0);
  load_sblk(S[1], lr, min(1, last_blk));
  load_wset<BITS>(W[0], lr, 0);
  load_wset<BITS>(W[1], lr, min(1, last));
  load_wset<BITS>(W[2], lr, min(2, last));
  // activations: two groups ahead when registers allow, else one
  constexpr int XD = NMB > 4 ? 1 : 2;
  stage_load<NMB>(rows, 0, X[0]);
  stage_store<NMB>(lds, X[0]);
  if constexpr (XD == 2) stage_load<NMB>(rows, min(1, last), X[1]);
#pragma unroll
  for (int jb = 0; jb < 16; ++jb) dequant_job<BITS>(W[0], S[0], 0, jb, B0[0], B1[0]);
  __syncthreads();

  for (int j0 = 0; j0 < n_groups; j0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u;
      load_wset<BITS>(W[(u + 3) & 3], lr, min(j + 3, last));
      if constexpr (XD == 2)
        stage_load<NMB>(rows, min(j + 2, last), X[u & 1]);
      else
        stage_load<NMB>(rows, min(j + 1, last), X[0]);
      const uint16_t* xs = lds + (u & 1) * (kTileM * kLdsRow) + m * kLdsRow + 32 * h;
      // Fragment f = (mb, st): two MFMAs (gate/up or two down rows).  The
      // next group's dequant is spread over the fragments and the LDS
      // reads run two fragments ahead; sched_barrier keeps that order.
      constexpr int NF = 4 * NMB;
      const SBlk& sn = u < 7 ? S[0] : S[1];
      const int si = (u + 1) & 7;
      bf16x8 A[3];
      A[0] = *reinterpret_cast<const bf16x8*>(xs);
      if constexpr (NF > 1) A[1] = *reinterpret_cast<const bf16x8*>(xs + 8);
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        if (f + 2 < NF)
          A[(f + 2) % 3] = *reinterpret_cast<const bf16x8*>(
              xs + ((f + 2) >> 2) * 32 * kLdsRow + 8 * ((f + 2) & 3));
        acc0[f >> 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[f % 3], B0[u & 1][f & 3],
                                                               acc0[f >> 2], 0, 0, 0);
        acc1[f >> 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[f % 3], B1[u & 1][f & 3],
                                                               acc1[f >> 2], 0, 0, 0);
#pragma unroll
        for (int jb = 16 * f / NF; jb < 16 * (f + 1) / NF; ++jb)
          dequant_job<BITS>(W[(u + 1) & 3], sn, si, jb, B0[(u + 1) & 1], B1[(u + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      stage_store<NMB>(lds + ((u + 1) & 1) * (kTileM * kLdsRow), X[XD == 2 ? (u + 1) & 1 : 0]);
      if (u == 7) {
        S[0] = S[1];
        load_sblk(S[1], lr, min((j0 >> 3) + 2, last_blk));
      }
      __syncthreads();
    }
  }
}

// Row of accumulator register r of a 32x32 block for lane half h.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

template <int BITS>
__device__ __forceinline__ void gemm_tile_any(int nmb, int n_groups, const StageRows& rows,
                                              const LaneRows& lr, uint16_t* lds,
                                              f32x16 (&acc0)[kMB], f32x16 (&acc1)[kMB]) {
  switch (nmb) {
    case 1: gemm_tile<BITS, 1>(n_groups, rows, lr, lds, acc0, acc1); break;
    case 2: gemm_tile<BITS, 2>(n_groups, rows, lr, lds, acc0, acc1); break;
    case 3: gemm_tile<BITS, 3>(n_groups, rows, lr, lds, acc0, acc1); break;
    case 4: gemm_tile<BITS, kMB >= 4 ? 4 : 1>(n_groups, rows, lr, lds, acc0, acc1); break;
    case 5: gemm_tile<BITS, kMB >= 5 ? 5 : 1>(n_groups, rows, lr, lds, acc0, acc1); break;
    case 6: gemm_tile<BITS, kMB >= 6 ? 6 : 1>(n_groups, rows, lr, lds, acc0, acc1); break;
    case 7: gemm_tile<BITS, kMB >= 7 ? 7 : 1>(n_groups, rows, lr, lds, acc0, acc1); break;
    default: gemm_tile<BITS, kMB>(n_groups, rows, lr, lds, acc0, acc1); break;
  }
}

// Blocks are dealt to the 8 XCDs round-robin by linear id; remap so each XCD
// gets a contiguous run of (tile, column block) work items: the column blocks
// of one tile share its activation rows, and consecutive tiles of one expert
// share weights, in that XCD's L2.  The grid is a multiple of 8 blocks and at
// least 8 * ceil(total / 8), so every item has a block.  Returns false for
// blocks with no work.
__device__ __forceinline__ bool xcd_work(int n_cols, int n_tiles, int& tile, int& cb) {
  const int total = n_cols * n_tiles;
  const int lin = blockIdx.x + gridDim.x * blockIdx.y;
  const int per = (total + 7) >> 3;
  const int w = (lin & 7) * per + (lin >> 3);
  if ((lin >> 3) >= per || w >= total) return false;
  tile = w / n_cols;
  cb = w - tile * n_cols;
  return true;
}

// ---------------------------------------------------------------- kernels

template <int BITS>
__global__ __launch_bounds__(kThreads) void gateup_mfma_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kTileM * kLdsRow];
  int t, cb;
  if (!xcd_work(a.out_cols / kGuCols, *a.n_tiles, t, cb)) return;
  const TileInfo ti = tile_info(a, t);
  if (ti.slot < 0) return;  // the down kernel writes this tile's zero rows
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = cb * kGuCols + wave * 32 + (lane & 31);
  const uint8_t* base = a.slab + size_t(ti.slot) * size_t(a.expert_bytes);
  const size_t row_bytes = size_t(a.cols) * BITS / 8;
  const int groups = a.cols / 64;
  constexpr int kHalf = 64 * BITS / 16;  // bytes of half a group
  const int h = lane >> 5;
  StageRows rows;
  rows.base = a.act;
#pragma unroll
  for (int j = 0; j < kMB; ++j) {
    const int r = min(32 * j + int(threadIdx.x >> 3), ti.m - 1);
    rows.off[j] = uint32_t(a.order[ti.p0 + r] / a.kk) * uint32_t(a.cols);
  }
  const u32x4* sp0 = reinterpret_cast<const u32x4*>(base + a.s0);
  const u32x4* bp0 = reinterpret_cast<const u32x4*>(base + a.b0);
  const u32x4* sp1 = reinterpret_cast<const u32x4*>(base + a.s1);
  const u32x4* bp1 = reinterpret_cast<const u32x4*>(base + a.b1);
  const int blks = groups / 8;
  LaneRows lr;
  lr.w0 = base + a.w0 + col * row_bytes + h * kHalf;
  lr.w1 = base + a.w1 + col * row_bytes + h * kHalf;
  lr.s0 = sp0 + size_t(col) * blks;
  lr.b0 = bp0 + size_t(col) * blks;
  lr.s1 = sp1 + size_t(col) * blks;
  lr.b1 = bp1 + size_t(col) * blks;
  f32x16 accg[kMB], accu[kMB];
  const int nmb = (ti.m + 31) >> 5;
  gemm_tile_any<BITS>(nmb, groups, rows, lr, lds, accg, accu);
  uint16_t* hout = static_cast<uint16_t*>(a.out);
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
  int t, cb;
  if (!xcd_work(a.out_cols / kDnCols, *a.n_tiles, t, cb)) return;
  const TileInfo ti = tile_info(a, t);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col0 = cb * kDnCols + wave * 64 + (lane & 31);
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
  constexpr int kHalf = 64 * BITS / 16;
  StageRows rows;
  rows.base = a.act;
#pragma unroll
  for (int j = 0; j < kMB; ++j) {
    const int r = min(32 * j + int(threadIdx.x >> 3), ti.m - 1);
    rows.off[j] = uint32_t(ti.p0 + r) * uint32_t(a.cols);
  }
  const u32x4* sp = reinterpret_cast<const u32x4*>(base + a.s0);
  const u32x4* bp = reinterpret_cast<const u32x4*>(base + a.b0);
  const int blks = groups / 8;
  LaneRows lr;
  lr.w0 = base + a.w0 + col0 * row_bytes + h * kHalf;
  lr.w1 = base + a.w0 + col1 * row_bytes + h * kHalf;
  lr.s0 = sp + size_t(col0) * blks;
  lr.b0 = bp + size_t(col0) * blks;
  lr.s1 = sp + size_t(col1) * blks;
  lr.b1 = bp + size_t(col1) * blks;
  f32x16 acc0[kMB], acc1[kMB];
  const int nmb = (ti.m + 31) >> 5;
  gemm_tile_any<BITS>(nmb, groups, rows, lr, lds, acc0, acc1);
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
  // column blocks must tile the outputs; the pipeline runs 4 groups per trip
  // scales are read 8 groups (16 bytes) at a time
  if (g->inter % kGuCols || g->hidden % kDnCols || g->inter % 512 || g->hidden % 512) return false;
  return rows >= 1024 && rows >= 16L * n_ids;
}

int prefill_experts(const pmoe_geom* g, const uint8_t* slab, const int32_t* table, int n_experts,
                    int shared_slot, const uint16_t* x, int n, int kk, const int32_t* order,
                    const int32_t* counts, const int32_t* offsets, const int2* tiles,
                    const int32_t* n_tiles, int max_tiles, uint16_t* h, void* y, int y_f32,
                    hipStream_t st) {
  PMOE_REQUIRE(g->inter % 512 == 0 && g->hidden % 512 == 0,
               "prefill: hidden and inter must be multiples of 512");
  PMOE_REQUIRE(max_tiles > 0 && max_tiles <= (1 << 20), "prefill: tile count out of range");
  PMOE_REQUIRE(int64_t(n) * g->hidden < (int64_t(1) << 31) &&
                   int64_t(n) * kk * g->inter < (int64_t(1) << 31),
               "prefill: activations exceed 2^31 elements");
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
    const int items = g->inter / kGuCols * max_tiles;
    dim3 grid((items + 7) / 8 * 8);  // a multiple of 8: xcd_work deals items per XCD
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
    const int items = g->hidden / kDnCols * max_tiles;
    dim3 grid((items + 7) / 8 * 8);
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
