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
// Work split (512 threads = 8 waves, two per SIMD): the tile's activation
// rows are staged through LDS one 64-wide quantization group at a time
// (double buffered) and shared by the 8 waves; each wave owns 32 weight rows
// (32 gate rows, 32 up rows, or 32 down rows: lane m of either lane half
// holds row m), loads their packed words straight from HBM, and dequantizes
// them in registers into the MFMA B operand, so every weight byte is read and
// dequantized once per tile.  One projection per wave keeps a wave within
// 256 registers (64 accumulators), so two waves share each SIMD and one
// covers the other's memory waits and dequant; the gate/up kernel pairs gate
// wave w with up wave w + 4 (the same rows and columns) through LDS for the
// SwiGLU.  v_mfma_f32_32x32x16_bf16, fp32 accumulators.  The dequantized
// weight is bf16(fma(s, q, b)), the format's bf16 dequantization
// (quant.hip), like the bf16 tile loads of mlx's quantized GEMMs.
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
constexpr int kLdsRow2 = 136;        // two groups a row (128 + 8 pad: 272 B)
constexpr int kThreads = 512;
constexpr int kStageSteps = kTileM * 8 / kThreads;  // 16-byte pieces per thread per group
constexpr int kGuCols = 128;         // moe_intermediate columns per gate/up block
constexpr int kDnCols = 256;         // hidden columns per down block

struct PrefillArgs {
  const uint8_t* slab;
  int64_t expert_bytes;
  const int32_t* order;
  const int4* tiles;     // {slot, first row, expert rows, expert offset} per tile
  const int32_t* n_tiles;
  const uint16_t* act;   // gate/up: x [n, hidden]; down: h [rows, inter] in sorted order
  int kk;                // flat rows per token (gate/up activation gather)
  int cols;              // reduction length: hidden (gate/up) or inter (down)
  int64_t w0, s0, b0;    // component offsets of the first weight matrix
  int64_t w1, s1, b1;    // and of the second (up for gate/up; = first for down)
  int out_cols;          // inter (h) or hidden (y)
  void* out;
  int out_f32;
  int out_vec;           // out is 16-byte aligned: bf16 rows may go out as 16-byte pieces
};

// Tile of this block: first sorted position, row count, slot.
struct TileInfo {
  int p0, m, slot;
};


// ---------------------------------------------------------------- dequant

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }

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

// bf16 pair (a in the low half, b in the high half) in one word: one
// v_cvt_pk_bf16_f32, rounding each to nearest even like a bf16 cast.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// Half HF (values 4*HF .. 4*HF+3) of one 4-bit word, lo = w & 0x0F0F0F0F
// (even values), hi = (w >> 4) & 0x0F0F0F0F (odd values), into words
// o[2HF], o[2HF+1] of the operand (two bf16 each).
template <int HF>
__device__ __forceinline__ void deq4_half(uint32_t lo, uint32_t hi, float s, float b,
                                          u32x4& o) {
  o[2 * HF] = pk_bf16(__builtin_fmaf(s, ubyte_f<2 * HF>(lo), b),
                      __builtin_fmaf(s, ubyte_f<2 * HF>(hi), b));
  o[2 * HF + 1] = pk_bf16(__builtin_fmaf(s, ubyte_f<2 * HF + 1>(lo), b),
                          __builtin_fmaf(s, ubyte_f<2 * HF + 1>(hi), b));
}

// 6-bit field J of a little-endian bit stream held in words w[], as float:
// one v_bfe_u32 (or, across a word boundary, v_alignbit_b32 and a mask)
// and one v_cvt_f32_ubyte0.
template <int J>
__device__ __forceinline__ float field6f(const uint32_t* w) {
  constexpr int bit = 6 * J, wi = bit / 32, sh = bit % 32;
  uint32_t v;
  if constexpr (sh <= 26)
    v = (w[wi] >> sh) & 63u;
  else
    v = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & 63u;
  return float(v);
}

// Values 8S + 4HF .. 8S + 4HF + 3 of a 6-bit half group into words
// o[2HF], o[2HF+1] of the operand.
template <int S, int HF>
__device__ __forceinline__ void deq4_6(const uint32_t* w, float s, float b, u32x4& o) {
  constexpr int J = 8 * S + 4 * HF;
  o[2 * HF] = pk_bf16(__builtin_fmaf(s, field6f<J>(w), b), __builtin_fmaf(s, field6f<J + 1>(w), b));
  o[2 * HF + 1] =
      pk_bf16(__builtin_fmaf(s, field6f<J + 2>(w), b), __builtin_fmaf(s, field6f<J + 3>(w), b));
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

// ---------------------------------------------------------------- staging

// One group (64 values) of the tile's activation rows -> registers.
// Piece p = kThreads*j + t (j < kStageSteps) of the 16-byte pieces is row
// p / 8, chunk p % 8, so each load instruction covers whole 128-byte row
// segments.  Rows past the tile re-load the tile's last row: every load
// stays in bounds and the code has no branch; the MFMA rows they feed are
// never stored.
struct StageRows {
  const uint16_t* base;
  uint32_t off[kStageSteps];  // element offset of each staged row
};

struct StageRegs {
  u32x4 v[kStageSteps];
};

// Only the pieces of the first NMB 32-row blocks are staged.
template <int NMB>
constexpr int stage_steps() {
  return (32 * NMB * 8 + kThreads - 1) / kThreads;
}

template <int NMB>
__device__ __forceinline__ void stage_load(const StageRows& sr, int g, StageRegs& x) {
  const int c = threadIdx.x & 7;
#pragma unroll
  for (int j = 0; j < stage_steps<NMB>(); ++j)
    x.v[j] = *reinterpret_cast<const u32x4*>(sr.base + sr.off[j] + g * 64 + c * 8);
}

template <int NMB, int PITCH = kLdsRow>
__device__ __forceinline__ void stage_store(uint16_t* lds, const StageRegs& x) {
  const int c = threadIdx.x & 7;
  const int r0 = threadIdx.x >> 3;
#pragma unroll
  for (int j = 0; j < stage_steps<NMB>(); ++j)
    *reinterpret_cast<u32x4*>(lds + ((kThreads / 8) * j + r0) * PITCH + c * 8) = x.v[j];
}

// ---------------------------------------------------------------- main loop

// The lane's weight row (half of each group: lane half h) with its scale and
// bias rows (bf16, one per group, read 8 groups at a time).
struct LaneRow {
  const uint8_t* w;
  const u32x4* s;
  const u32x4* b;
};

// Scales and biases of 8 consecutive groups.
struct SBlk {
  u32x4 s, b;
};

template <int BITS>
__device__ __forceinline__ void load_group(LaneWords<BITS>& lw, const LaneRow& lr, int g) {
  constexpr int kGroupBytes = 64 * BITS / 8;
  load_words<BITS>(lw, lr.w + size_t(g) * kGroupBytes);
}

__device__ __forceinline__ void load_sblk(SBlk& sb, const LaneRow& lr, int blk) {
  sb.s = lr.s[blk];
  sb.b = lr.b[blk];
}

// bf16 entry i (0..7) of 8 packed in a u32x4, as float.
__device__ __forceinline__ float bf_at(const u32x4& v, int i) {
  const uint32_t w = v[i >> 1];
  return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
}

// Dequant job jb (0..7) of a group: half jb & 1 (4 values) of MFMA step
// jb >> 1, with the group's scale/bias at entry i of sb.  Eight small jobs
// per group let the dequant spread evenly between the MFMAs.  The operand
// of step st is o[st]: 8 bf16 as 4 words.
template <int BITS>
__device__ __forceinline__ void dequant_job(const LaneWords<BITS>& lw, const SBlk& sb, int i,
                                            int jb, u32x4 (&o)[4]) {
  const int st = jb >> 1;
  const float s = bf_at(sb.s, i);
  const float b = bf_at(sb.b, i);
  u32x4& out = o[st];
  if constexpr (BITS == 4) {
    const uint32_t w = lw.w[st];
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    if (jb & 1)
      deq4_half<1>(lo, hi, s, b, out);
    else
      deq4_half<0>(lo, hi, s, b, out);
  } else {
    switch (jb) {
      case 0: deq4_6<0, 0>(lw.w, s, b, out); break;
      case 1: deq4_6<0, 1>(lw.w, s, b, out); break;
      case 2: deq4_6<1, 0>(lw.w, s, b, out); break;
      case 3: deq4_6<1, 1>(lw.w, s, b, out); break;
      case 4: deq4_6<2, 0>(lw.w, s, b, out); break;
      case 5: deq4_6<2, 1>(lw.w, s, b, out); break;
      case 6: deq4_6<3, 0>(lw.w, s, b, out); break;
      default: deq4_6<3, 1>(lw.w, s, b, out); break;
    }
  }
}

// LDS rows of one activation staging buffer: the tile's rows, and at least
// the 64 rows one staging step of 512 threads writes.
template <int MB>
constexpr int stage_rows() {
  return 32 * MB > 64 ? 32 * MB : 64;
}

// One group's MFMAs for the tile's first NMB 32-row blocks (activations at
// xs in LDS, weights b), with the next group's dequant (words wn, scale and
// bias entry si of sn, into bn) spread over the fragments.  Fragment
// f = (mb, st): one MFMA; the LDS reads run two fragments ahead, and
// sched_barrier keeps that order.  (Step-major order, with consecutive
// MFMAs on different accumulators, measured slower: the second wave on the
// SIMD already fills the accumulation latency.)
template <int BITS, int NMB, int MB, int PITCH = kLdsRow>
__device__ __forceinline__ void group_mfma(const uint16_t* xs, const u32x4 (&b)[4],
                                           const LaneWords<BITS>& wn, const SBlk& sn, int si,
                                           u32x4 (&bn)[4], f32x16 (&acc)[MB]) {
  constexpr int NF = 4 * NMB;
  bf16x8 A[3];
  A[0] = *reinterpret_cast<const bf16x8*>(xs);
  if constexpr (NF > 1) A[1] = *reinterpret_cast<const bf16x8*>(xs + 8);
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    if (f + 2 < NF)
      A[(f + 2) % 3] = *reinterpret_cast<const bf16x8*>(
          xs + ((f + 2) >> 2) * 32 * PITCH + 8 * ((f + 2) & 3));
    acc[f >> 2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        A[f % 3], __builtin_bit_cast(bf16x8, b[f & 3]), acc[f >> 2], 0, 0, 0);
#pragma unroll
    for (int jb = 8 * f / NF; jb < 8 * (f + 1) / NF; ++jb) dequant_job<BITS>(wn, sn, si, jb, bn);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// acc[mb] = A_tile(mb) . B over the whole reduction, for the tile's first
// NMB 32-row blocks.  Software pipeline (per quantization group j): weights
// of group j+WD (3, or 7 for an 8-group reduction: all of them) and
// activations of group j+2 are in flight, group j+1's
// weights are dequantized while group j's MFMAs run, and group j+1's
// activations go to the other LDS buffer.  Scales/biases arrive 8 groups at
// a time, one block ahead.  The loop is unrolled by 8 so the register rings
// are indexed statically; loads past the end clamp to the last group (their
// data is unused).  n_groups is a multiple of 8.
template <int BITS, int NMB, int MB, int WD = 3>
__device__ __forceinline__ void gemm_tile(int n_groups, const StageRows& rows, const LaneRow& lr,
                                          uint16_t* lds, f32x16 (&acc)[MB]) {
  static_assert(NMB <= MB, "row blocks beyond the accumulators");
  static_assert(WD == 3 || WD == 7, "weight groups in flight: a ring of 4 or 8");
  constexpr int WR = WD + 1;
  constexpr int SR = stage_rows<MB>();
  const int lane = threadIdx.x & 63;
  const int m = lane & 31;
  const int h = lane >> 5;
  const int last = n_groups - 1;
  const int last_blk = (n_groups >> 3) - 1;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16{};
  LaneWords<BITS> W[WR];
  StageRegs X[2];
  SBlk S[2];
  u32x4 B[2][4];
  load_sblk(S[0], lr, 0);
  load_sblk(S[1], lr, min(1, last_blk));
#pragma unroll
  for (int i = 0; i < WD; ++i) load_group<BITS>(W[i], lr, min(i, last));
  stage_load<NMB>(rows, 0, X[0]);
  stage_store<NMB>(lds, X[0]);
  stage_load<NMB>(rows, min(1, last), X[1]);
#pragma unroll
  for (int jb = 0; jb < 8; ++jb) dequant_job<BITS>(W[0], S[0], 0, jb, B[0]);
  __syncthreads();

  for (int j0 = 0; j0 < n_groups; j0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u;
      load_group<BITS>(W[(u + WD) % WR], lr, min(j + WD, last));
      stage_load<NMB>(rows, min(j + 2, last), X[u & 1]);
      const uint16_t* xs = lds + (u & 1) * (SR * kLdsRow) + m * kLdsRow + 32 * h;
      group_mfma<BITS, NMB, MB>(xs, B[u & 1], W[(u + 1) % WR], u < 7 ? S[0] : S[1], (u + 1) & 7,
                                B[(u + 1) & 1], acc);
      stage_store<NMB>(lds + ((u + 1) & 1) * (SR * kLdsRow), X[(u + 1) & 1]);
      if (u == 7) {
        S[0] = S[1];
        load_sblk(S[1], lr, min((j0 >> 3) + 2, last_blk));
      }
      __syncthreads();
    }
  }
}

// 6-bit weights in coalesced units.  A lane's operand is half a group of
// one row (24 bytes); read straight from HBM, each load instruction would
// touch 32 rows for 512 bytes.  Instead a wave reads a unit -- 4 groups of
// its 32 rows, 192 contiguous bytes a row -- as 6 loads of 16 bytes a lane,
// copies it into its own LDS buffer (row pitch 200 bytes: the 8-byte reads
// of 16 consecutive rows fall on distinct banks) and reads each group's
// half rows back in the operand layout.  The words are the same, so the
// dequant and the MFMAs (and their results) are unchanged.
//
// Rows are whole 128-byte lines (their length is a multiple of 384 bytes),
// so units k and k + 1 (k even) of a row share the line of bytes
// [192 k + 128, 192 k + 256).  The pieces a row owns outright (8 of its
// 12: the unit's whole line) are loaded by 4 instructions of 8 rows x 128
// bytes, non-temporal; the shared half line (4 pieces) by 2 instructions
// of 16 rows x 64 bytes, cached, so that the unit 4 groups later can find
// it in L2 instead of reading the line from HBM a second time.
constexpr int kUnitPieces = 6;                  // 16-byte pieces a lane per unit
constexpr int kUnitPitch = 200;                 // LDS bytes per row of a unit
constexpr int kUnitLds = 32 * kUnitPitch;       // LDS bytes per wave

struct Unit6 {
  u32x4 v[kUnitPieces];
};

// Piece i (0..5) of a lane in a unit of parity P: its row r and 16-byte
// column c (0..11) within the row's 192 bytes.  Pieces 0-3: the unit's own
// line (columns 0-7, or 4-11 for odd units); 4-5: the shared half line
// (columns 8-11, or 0-3).
template <int P>
__device__ __forceinline__ void unit_piece(int i, uint32_t lane, uint32_t& r, uint32_t& c) {
  if (i < 4) {
    r = 8 * i + (lane >> 3);
    c = (lane & 7) + 4 * P;
  } else {
    r = 16 * (i - 4) + (lane >> 2);
    c = (lane & 3) + 8 * (1 - P);
  }
}

// Unit k (parity P) of the wave's 32 rows into un (row 0 at w0, row_bytes
// apart; w0 is the same in every lane, so each load takes it as a scalar
// base with a 32-bit lane offset).
template <int P>
__device__ __forceinline__ void load_unit6(Unit6& un, const uint8_t* w0, uint32_t row_bytes,
                                           int k, uint32_t lane) {
  const uint8_t* wk = w0 + 192 * k;
#pragma unroll
  for (int i = 0; i < kUnitPieces; ++i) {
    uint32_t r, c;
    unit_piece<P>(i, lane, r, c);
    const u32x4* src = reinterpret_cast<const u32x4*>(wk + (r * row_bytes + 16 * c));
    if (i < 4)
      un.v[i] = __builtin_nontemporal_load(src);
    else
      un.v[i] = *src;
  }
}

// Copy the unit held in un (parity P) to buf, then (if load) load unit k
// (parity 1 - P) into un.
template <int P>
__device__ __forceinline__ void cycle_unit6(Unit6& un, uint8_t* buf, const uint8_t* w0,
                                            uint32_t row_bytes, int k, bool load) {
  uint32_t lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));  // opaque: addresses recomputed here, not held across the loop
#pragma unroll
  for (int i = 0; i < kUnitPieces; ++i) {
    uint32_t r, c;
    unit_piece<P>(i, lane, r, c);
    uint32_t* q = reinterpret_cast<uint32_t*>(buf + r * kUnitPitch + 16 * c);
    *reinterpret_cast<u32x2*>(q) = u32x2{un.v[i][0], un.v[i][1]};
    *reinterpret_cast<u32x2*>(q + 2) = u32x2{un.v[i][2], un.v[i][3]};
  }
  __builtin_amdgcn_sched_barrier(0);  // the copy reads un before it is reloaded
  if (load) load_unit6<1 - P>(un, w0, row_bytes, k, lane);
}

// Group gi (0..3) of the unit at lds + rd, where rd is the lane's half row
// in the wave's buffer (the same register for every group: the group's
// place is the instructions' offset field).
__device__ __forceinline__ void read_group6(LaneWords<6>& lw, const uint8_t* lds, uint32_t rd,
                                            int gi) {
  const u32x2* s = reinterpret_cast<const u32x2*>(lds + rd + 48 * gi);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const u32x2 t = s[j];
    lw.w[2 * j] = t[0];
    lw.w[2 * j + 1] = t[1];
  }
}

// gemm_tile for 6-bit weights read in units: the same pipeline, with the
// weights of group j+1 read from the wave's LDS copy of their unit.  One
// unit is held in registers: when group j+1 opens a unit, that unit is
// copied to LDS and its registers take the next one (4 groups ahead; a
// block's 16 waves keep ~96 KB a CU in flight).  n_groups is a multiple
// of 8.
template <int NMB, int MB>
__device__ __forceinline__ void gemm_tile_u6(int n_groups, const StageRows& rows,
                                             const uint8_t* w0, uint32_t row_bytes,
                                             const LaneRow& lr, uint16_t* lds, uint8_t* wbuf,
                                             f32x16 (&acc)[MB]) {
  static_assert(NMB <= MB, "row blocks beyond the accumulators");
  constexpr int SR = stage_rows<MB>();
  const int lane = threadIdx.x & 63;
  const int m = lane & 31;
  const int h = lane >> 5;
  const int last = n_groups - 1;
  const int last_blk = (n_groups >> 3) - 1;
  const int last_unit = (n_groups >> 2) - 1;
  const uint8_t* lds8 = reinterpret_cast<const uint8_t*>(lds);
  uint32_t rd = uint32_t(wbuf - lds8) + m * kUnitPitch + 24 * h;
  asm volatile("" : "+v"(rd));  // one base register for every group's reads
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16{};
  Unit6 U;
  LaneWords<6> Wn;
  StageRegs X[2];
  SBlk S[2];
  u32x4 B[2][4];
  load_sblk(S[0], lr, 0);
  load_sblk(S[1], lr, min(1, last_blk));
  load_unit6<0>(U, w0, row_bytes, 0, threadIdx.x & 63);
  stage_load<NMB>(rows, 0, X[0]);
  stage_store<NMB>(lds, X[0]);
  stage_load<NMB>(rows, min(1, last), X[1]);
  cycle_unit6<0>(U, wbuf, w0, row_bytes, 1, true);
  read_group6(Wn, lds8, rd, 0);
#pragma unroll
  for (int jb = 0; jb < 8; ++jb) dequant_job<6>(Wn, S[0], 0, jb, B[0]);
  __syncthreads();

  for (int j0 = 0; j0 < n_groups; j0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u;
      // group j+1 opens unit un (held in U; odd at u = 3, even at u = 7)
      const int un = (j + 1) >> 2;
      if (u == 3 && un <= last_unit)
        cycle_unit6<1>(U, wbuf, w0, row_bytes, un + 1, un + 1 <= last_unit);
      if (u == 7 && un <= last_unit)
        cycle_unit6<0>(U, wbuf, w0, row_bytes, un + 1, un + 1 <= last_unit);
      read_group6(Wn, lds8, rd, (u + 1) & 3);
      stage_load<NMB>(rows, min(j + 2, last), X[u & 1]);
      const uint16_t* xs = lds + (u & 1) * (SR * kLdsRow) + m * kLdsRow + 32 * h;
      group_mfma<6, NMB, MB>(xs, B[u & 1], Wn, u < 7 ? S[0] : S[1], (u + 1) & 7,
                             B[(u + 1) & 1], acc);
      stage_store<NMB>(lds + ((u + 1) & 1) * (SR * kLdsRow), X[(u + 1) & 1]);
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

// 4-bit weights in units of 4 groups: one 128-byte line of each of the
// wave's 32 rows.  A unit is loaded as 4 instructions of 8 rows x 128
// bytes (lane l: row 8 i + l / 8, 16-byte column l % 8), non-temporal
// since no line is read again, copied to the wave's LDS buffer (row pitch
// 144 bytes: the 16-byte reads of 16 consecutive rows fall on distinct
// banks), and each group's half row is read back in the operand layout
// (16 bytes a lane, where the direct form loaded them from HBM with each
// instruction touching 32 rows).  Same words, same results.
constexpr int kUnit4Pitch = 144;
constexpr int kUnit4Lds = 32 * kUnit4Pitch;  // LDS bytes per wave

struct Unit4 {
  u32x4 v[4];
};

__device__ __forceinline__ void load_unit4(Unit4& un, const uint8_t* w0, uint32_t row_bytes, int k,
                                           uint32_t lane) {
  const uint8_t* wk = w0 + 128 * k;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    un.v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
        wk + ((8 * i + (lane >> 3)) * row_bytes + 16 * (lane & 7))));
}

// Copy the unit held in un to buf, then (if load) load unit k into un.
__device__ __forceinline__ void cycle_unit4(Unit4& un, uint8_t* buf, const uint8_t* w0,
                                            uint32_t row_bytes, int k, bool load) {
  uint32_t lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));  // opaque: addresses recomputed here, not held across the loop
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<u32x4*>(buf + (8 * i + (lane >> 3)) * kUnit4Pitch + 16 * (lane & 7)) =
        un.v[i];
  __builtin_amdgcn_sched_barrier(0);  // the copy reads un before it is reloaded
  if (load) load_unit4(un, w0, row_bytes, k, lane);
}

// Group gi (0..3) of the unit at lds + rd (rd: the lane's half row).
__device__ __forceinline__ void read_group4(LaneWords<4>& lw, const uint8_t* lds, uint32_t rd,
                                            int gi) {
  const u32x4 t = *reinterpret_cast<const u32x4*>(lds + rd + 32 * gi);
  lw.w[0] = t[0];
  lw.w[1] = t[1];
  lw.w[2] = t[2];
  lw.w[3] = t[3];
}

// gemm_tile for 4-bit weights read in units (128-row tiles): the same
// pipeline, the weights of group j+1 read from the wave's LDS copy of
// their unit; one unit in registers, loaded when the previous one is
// copied (4 groups ahead).  The activations are staged two groups at a time
// (rows of 272 bytes: both groups and 16 bytes of pad, conflict-free for the
// 16-byte fragment reads), so one block barrier serves two groups: pair p
// of groups sits in buffer p & 1, the pair after next is requested at the
// start of a pair and the next pair stored at its end (one group a barrier
// measured 1.5% slower over the 2048-token layer).  n_groups is a multiple
// of 8.
template <int NMB, int MB>
__device__ __forceinline__ void gemm_tile_u4(int n_groups, const StageRows& rows,
                                              const uint8_t* w0, uint32_t row_bytes,
                                              const LaneRow& lr, uint16_t* lds, uint8_t* wbuf,
                                              f32x16 (&acc)[MB]) {
  static_assert(NMB <= MB, "row blocks beyond the accumulators");
  constexpr int SR = stage_rows<MB>();
  constexpr int P = kLdsRow2;
  const int lane = threadIdx.x & 63;
  const int m = lane & 31;
  const int h = lane >> 5;
  const int last = n_groups - 1;
  const int last_blk = (n_groups >> 3) - 1;
  const int last_unit = (n_groups >> 2) - 1;
  const uint8_t* lds8 = reinterpret_cast<const uint8_t*>(lds);
  uint32_t rd = uint32_t(wbuf - lds8) + m * kUnit4Pitch + 16 * h;
  asm volatile("" : "+v"(rd));  // one base register for every group's reads
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16{};
  Unit4 U;
  LaneWords<4> Wn;
  StageRegs X[2][2];
  SBlk S[2];
  u32x4 B[2][4];
  load_sblk(S[0], lr, 0);
  load_sblk(S[1], lr, min(1, last_blk));
  load_unit4(U, w0, row_bytes, 0, threadIdx.x & 63);
  stage_load<NMB>(rows, 0, X[0][0]);
  stage_load<NMB>(rows, min(1, last), X[0][1]);
  stage_store<NMB, P>(lds, X[0][0]);
  stage_store<NMB, P>(lds + 64, X[0][1]);
  stage_load<NMB>(rows, min(2, last), X[1][0]);
  stage_load<NMB>(rows, min(3, last), X[1][1]);
  cycle_unit4(U, wbuf, w0, row_bytes, 1, true);
  read_group4(Wn, lds8, rd, 0);
#pragma unroll
  for (int jb = 0; jb < 8; ++jb) dequant_job<4>(Wn, S[0], 0, jb, B[0]);
  __syncthreads();

  for (int j0 = 0; j0 < n_groups; j0 += 8) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // pair q of this 8-group trip: groups j0 + 2q, j0 + 2q + 1 in buffer q & 1
      stage_load<NMB>(rows, min(j0 + 2 * q + 4, last), X[q & 1][0]);
      stage_load<NMB>(rows, min(j0 + 2 * q + 5, last), X[q & 1][1]);
      const uint16_t* xs = lds + (q & 1) * (SR * P) + m * P + 32 * h;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int u = 2 * q + v;
        const int j = j0 + u;
        // group j+1 opens unit un (held in U)
        const int un = (j + 1) >> 2;
        if ((u & 3) == 3 && un <= last_unit)
          cycle_unit4(U, wbuf, w0, row_bytes, un + 1, un + 1 <= last_unit);
        read_group4(Wn, lds8, rd, (u + 1) & 3);
        group_mfma<4, NMB, MB, P>(xs + 64 * v, B[u & 1], Wn, u < 7 ? S[0] : S[1], (u + 1) & 7,
                                  B[(u + 1) & 1], acc);
        if (u == 7) {
          S[0] = S[1];
          load_sblk(S[1], lr, min((j0 >> 3) + 2, last_blk));
        }
      }
      stage_store<NMB, P>(lds + ((q + 1) & 1) * (SR * P), X[(q + 1) & 1][0]);
      stage_store<NMB, P>(lds + ((q + 1) & 1) * (SR * P) + 64, X[(q + 1) & 1][1]);
      __syncthreads();
    }
  }
}

template <int BITS, int MB>
__device__ __forceinline__ void gemm_tile_any(int nmb, int n_groups, const StageRows& rows,
                                              const LaneRow& lr, const uint8_t* w0,
                                              uint32_t row_bytes, uint16_t* lds, uint8_t* wbuf,
                                              f32x16 (&acc)[MB]) {
  if constexpr (MB == 1 && BITS == 6) {
    gemm_tile_u6<1, 1>(n_groups, rows, w0, row_bytes, lr, lds, wbuf, acc);
  } else if constexpr (MB == 1) {
    // a reduction of 8 groups (a 512-wide down): every group's weights are
    // requested before the first MFMA
    if (n_groups == 8)
      gemm_tile<BITS, 1, 1, 7>(n_groups, rows, lr, lds, acc);
    else
      gemm_tile<BITS, 1, 1>(n_groups, rows, lr, lds, acc);
  } else if constexpr (BITS == 4) {
    switch (nmb) {
      case 1: gemm_tile_u4<1, MB>(n_groups, rows, w0, row_bytes, lr, lds, wbuf, acc); break;
      case 2: gemm_tile_u4<2, MB>(n_groups, rows, w0, row_bytes, lr, lds, wbuf, acc); break;
      case 3: gemm_tile_u4<3, MB>(n_groups, rows, w0, row_bytes, lr, lds, wbuf, acc); break;
      default: gemm_tile_u4<MB, MB>(n_groups, rows, w0, row_bytes, lr, lds, wbuf, acc); break;
    }
  } else {
    switch (nmb) {
      case 1: gemm_tile<BITS, 1, MB>(n_groups, rows, lr, lds, acc); break;
      case 2: gemm_tile<BITS, 2, MB>(n_groups, rows, lr, lds, acc); break;
      case 3: gemm_tile<BITS, 3, MB>(n_groups, rows, lr, lds, acc); break;
      default: gemm_tile<BITS, MB, MB>(n_groups, rows, lr, lds, acc); break;
    }
  }
}

// Staged rows of a tile: rows [p0, p0 + m) of the sorted order, gathered
// from act row order[p] / kk (gate/up) or read in place (order null: down).
// Rows past the tile re-load its last row.
__device__ __forceinline__ StageRows tile_rows(const uint16_t* act, const int32_t* order, int kk,
                                               int cols, int p0, int m) {
  StageRows rows;
  rows.base = act;
#pragma unroll
  for (int j = 0; j < kStageSteps; ++j) {
    const int r = p0 + min((kThreads / 8) * j + int(threadIdx.x >> 3), m - 1);
    rows.off[j] = uint32_t(order ? order[r] / kk : r) * uint32_t(cols);
  }
  return rows;
}

// Blocks are dealt to the 8 XCDs round-robin by linear id; remap so each XCD
// gets a contiguous run of work items, and order an expert's items column
// block first, tile second: the blocks that read one weight column block
// for each of the expert's tiles are consecutive, so they run side by side
// on one XCD and its L2 can serve the weights to all but the first.  The
// expert's items are the same range [t0 * n_cols, (t0 + nt) * n_cols) in
// either order, found from the tile that tile-major order puts at the item.
// The grid is a multiple of 8 blocks and at least 8 * ceil(total / 8), so
// every item has a block.  Returns false for blocks with no work.
template <int TM>
__device__ __forceinline__ bool xcd_work(const PrefillArgs& a, int n_cols, TileInfo& ti,
                                         int& cb) {
  const int total = n_cols * *a.n_tiles;
  const int lin = blockIdx.x + gridDim.x * blockIdx.y;
  const int per = (total + 7) >> 3;
  const int w = (lin & 7) * per + (lin >> 3);
  if ((lin >> 3) >= per || w >= total) return false;
  const int tp = w / n_cols;
  const int4 tl = a.tiles[tp];                    // the tile record carries the expert's
  const int cnt = tl.z;                           // slot, rows and offset
  const int t0 = tp - tl.y / TM;                  // the expert's first tile
  const int nt = (cnt + TM - 1) / TM;             // and its tile count
  const int l = w - t0 * n_cols;
  cb = l / nt;
  const int r0 = (l - cb * nt) * TM;              // first row of this item's tile
  ti.m = min(TM, cnt - r0);
  ti.p0 = tl.w + r0;
  ti.slot = tl.x;
  return true;
}

// ---------------------------------------------------------------- kernels

// Tile height.  Tiles of 128 rows (MB = kMB row blocks) run at one block
// per CU (218 registers a wave, 64 of them accumulators); for layers whose
// experts see few rows each the dispatch cuts 32-row tiles instead (MB = 1,
// about 105 registers, two blocks per CU, which hide each other's load
// latency), so an expert with many rows (a shared expert's, say) spreads
// over many blocks.  The dispatch's tile height is 32 * MB; a tile is
// clamped to that height in xcd_work.  Both forms give every row the same
// MFMA sequence, so the outputs are bit-identical.
//
// LDS of one block: the activation staging buffers, reused after the main
// loop by the gate/up epilogue for the up waves' accumulators.
// 6-bit weights at 32-row tiles go through the 8 waves' unit buffers after
// that (gemm_tile_u6).
template <int BITS, int MB>
constexpr int stage_bytes() {
  return 2 * stage_rows<MB>() * (BITS == 4 && MB > 1 ? kLdsRow2 : kLdsRow) * 2;
}
template <int BITS, int MB>
constexpr int unit_wave_bytes() {
  return BITS == 6 && MB == 1 ? kUnitLds : BITS == 4 && MB > 1 ? kUnit4Lds : 0;
}
template <int BITS, int MB>
constexpr int unit_lds_bytes() {
  return (kThreads / 64) * unit_wave_bytes<BITS, MB>();
}
template <int BITS, int MB>
constexpr int gateup_lds_bytes() {
  constexpr int up = 4 * MB * 16 * 64 * 4;  // 4 up waves x accumulators
  return (stage_bytes<BITS, MB>() > up ? stage_bytes<BITS, MB>() : up) + unit_lds_bytes<BITS, MB>();
}
template <int BITS, int MB>
constexpr int down_lds_bytes() {
  return stage_bytes<BITS, MB>() + unit_lds_bytes<BITS, MB>();
}

template <int BITS, int MB>
__global__ __launch_bounds__(kThreads, MB < kMB ? 4 : 1) void gateup_mfma_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_raw[gateup_lds_bytes<BITS, MB>()];
  uint16_t* lds = reinterpret_cast<uint16_t*>(lds_raw);
  TileInfo ti;
  int cb;
  if (!xcd_work<32 * MB>(a, a.out_cols / kGuCols, ti, cb)) return;
  if (ti.slot < 0) return;  // the down kernel writes this tile's zero rows
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int up = wave >> 2;   // waves 0-3: gate rows, 4-7: the same up rows
  const int wq = wave & 3;
  const int col = cb * kGuCols + wq * 32 + (lane & 31);
  const uint8_t* base = a.slab + size_t(ti.slot) * size_t(a.expert_bytes);
  const size_t row_bytes = size_t(a.cols) * BITS / 8;
  const int groups = a.cols / 64;
  constexpr int kHalf = 64 * BITS / 16;  // bytes of half a group
  const int h = lane >> 5;
  const int blks = groups / 8;
  LaneRow lr;
  lr.w = base + (up ? a.w1 : a.w0) + col * row_bytes + h * kHalf;
  lr.s = reinterpret_cast<const u32x4*>(base + (up ? a.s1 : a.s0)) + size_t(col) * blks;
  lr.b = reinterpret_cast<const u32x4*>(base + (up ? a.b1 : a.b0)) + size_t(col) * blks;
  const int col0 = cb * kGuCols + wq * 32;  // the wave's first row (uniform)
  const uint8_t* w0 = base + (up ? a.w1 : a.w0) + size_t(col0) * row_bytes;
  uint8_t* wbuf = lds_raw + gateup_lds_bytes<BITS, MB>() - unit_lds_bytes<BITS, MB>() +
                  wave * unit_wave_bytes<BITS, MB>();
  const StageRows rows = tile_rows(a.act, a.order, a.kk, a.cols, ti.p0, ti.m);
  f32x16 acc[MB];
  const int nmb = (ti.m + 31) >> 5;
  gemm_tile_any<BITS, MB>(nmb, groups, rows, lr, w0, uint32_t(row_bytes), lds, wbuf, acc);
  // SwiGLU: gate wave wq and up wave wq + 4 hold the same rows and columns,
  // lane for lane, and swap halves through LDS (the staging buffers are
  // free: the main loop ended with a block barrier).  With several row
  // blocks each computes half of them (the up wave hands over the first
  // half, the gate wave the second); with one, the gate wave computes it.
  // h = silu(gate) * up either way.
  float* ul = reinterpret_cast<float*>(lds_raw);
  constexpr int kSplit = MB > 1 ? MB / 2 : MB;  // row blocks the gate wave computes
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    if (mb < nmb && (up ? mb < kSplit : mb >= kSplit))
#pragma unroll
      for (int r = 0; r < 16; ++r) ul[((wq * MB + mb) * 16 + r) * 64 + lane] = acc[mb][r];
  __syncthreads();
  uint16_t* hout = static_cast<uint16_t*>(a.out);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (up ? mb < kSplit : mb >= kSplit) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = mb * 32 + acc_row(r, h);
      if (row < ti.m) {
        const float o = ul[((wq * MB + mb) * 16 + r) * 64 + lane];
        const float g = up ? o : acc[mb][r];
        const float u = up ? acc[mb][r] : o;
        const float v = silu_fast(g) * u;
        hout[size_t(ti.p0 + row) * a.out_cols + col] = f2bf(v);
      }
    }
  }
  // (Staging h through an LDS tile after the exchange area and storing
  // 16-byte row pieces, as the down does, made gate/up slower at 128-row
  // tiles: 738 -> 748 us for the 2048-token layer in rocprof; the extra
  // block barrier costs more than 32 KB of short stores.)
}

template <int BITS, int MB>
__global__ __launch_bounds__(kThreads, MB < kMB ? 4 : 1) void down_mfma_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_raw[down_lds_bytes<BITS, MB>()];
  uint16_t* lds = reinterpret_cast<uint16_t*>(lds_raw);
  TileInfo ti;
  int cb;
  if (!xcd_work<32 * MB>(a, a.out_cols / kDnCols, ti, cb)) return;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = cb * kDnCols + wave * 32 + (lane & 31);
  const int h = lane >> 5;
  if (ti.slot < 0) {  // not resident: exact zero rows (streaming.py:715-719)
    for (int row = h; row < ti.m; row += 2) {
      const size_t o = size_t(a.order[ti.p0 + row]) * a.out_cols;
      if (a.out_f32)
        static_cast<float*>(a.out)[o + col] = 0.0f;
      else
        static_cast<uint16_t*>(a.out)[o + col] = 0;
    }
    return;
  }
  const uint8_t* base = a.slab + size_t(ti.slot) * size_t(a.expert_bytes);
  const size_t row_bytes = size_t(a.cols) * BITS / 8;
  const int groups = a.cols / 64;
  constexpr int kHalf = 64 * BITS / 16;
  const int blks = groups / 8;
  LaneRow lr;
  lr.w = base + a.w0 + col * row_bytes + h * kHalf;
  lr.s = reinterpret_cast<const u32x4*>(base + a.s0) + size_t(col) * blks;
  lr.b = reinterpret_cast<const u32x4*>(base + a.b0) + size_t(col) * blks;
  const int col0 = cb * kDnCols + wave * 32;  // the wave's first row (uniform)
  const uint8_t* w0 = base + a.w0 + size_t(col0) * row_bytes;
  uint8_t* wbuf = lds_raw + stage_bytes<BITS, MB>() + wave * unit_wave_bytes<BITS, MB>();
  const StageRows rows = tile_rows(a.act, nullptr, 1, a.cols, ti.p0, ti.m);
  // the tile's output rows, read while the weights stream (the main loop's
  // barriers publish them), not one dependent load per row at the end
  __shared__ int32_t s_ord[32 * MB];
  if (int(threadIdx.x) < ti.m) s_ord[threadIdx.x] = a.order[ti.p0 + threadIdx.x];
  f32x16 acc[MB];
  const int nmb = (ti.m + 31) >> 5;
  gemm_tile_any<BITS, MB>(nmb, groups, rows, lr, w0, uint32_t(row_bytes), lds, wbuf, acc);
  // bf16 rows go out through LDS (free: the main loop ended with a block
  // barrier) as 16-byte row pieces, 32 threads a row: 2-byte stores straight
  // from the accumulators, each instruction covering half a line of two
  // rows, took a fifth of a block's life.  Row pitch kDnCols + 8 values
  // (528 bytes): the rows the two lane halves write fall on other banks.
  // Forms whose LDS cannot hold the tile (6-bit, 128 rows) store directly.
  constexpr int kEp = kDnCols + 8;
  constexpr int kPieces = kDnCols / 8;
  constexpr bool kStaged = 32 * MB * kEp * 2 <= down_lds_bytes<BITS, MB>();
  if (!kStaged || a.out_f32 || !a.out_vec) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = mb * 32 + acc_row(r, h);
        if (row < ti.m) {
          const size_t o = size_t(s_ord[row]) * a.out_cols;
          if (a.out_f32)
            static_cast<float*>(a.out)[o + col] = acc[mb][r];
          else
            static_cast<uint16_t*>(a.out)[o + col] = f2bf(acc[mb][r]);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    if (mb < nmb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        lds[(mb * 32 + acc_row(r, h)) * kEp + wave * 32 + (lane & 31)] = f2bf(acc[mb][r]);
  __syncthreads();
  uint16_t* out = static_cast<uint16_t*>(a.out) + cb * kDnCols;
  for (int q = threadIdx.x; q < ti.m * kPieces; q += kThreads) {
    const int row = q / kPieces, pc = q - row * kPieces;
    *reinterpret_cast<uint4*>(out + size_t(s_ord[row]) * a.out_cols + 8 * pc) =
        *reinterpret_cast<const uint4*>(lds + row * kEp + 8 * pc);
  }
}

}  // namespace

// 32-row tiles at two blocks per CU when the routed experts see at most 32
// rows each on average (n * kk rows over n_experts); PMOE_PREFILL_SMALL=1 /
// 0 pins either form (read per call, so the two can be compared).
int prefill_tile_rows(int n, int kk, int n_experts) {
  const char* v = getenv("PMOE_PREFILL_SMALL");
  bool small = long(n) * kk <= 32L * n_experts;
  if (v && v[0] == '1') small = true;
  if (v && v[0] == '0') small = false;
  return small ? 32 : kTileM;
}

int prefill_min_tile_rows() { return 32; }

}  // namespace pmoe

extern "C" int pmoe_prefill_tile_rows(int n, int kk, int n_experts) {
  return pmoe::prefill_tile_rows(n, kk, n_experts);
}

namespace pmoe {

// The MFMA path pays off once experts see tens of rows; below that the
// weight-streaming GEMV (decode.hip) is as fast and needs no tile list.
bool prefill_wanted(const pmoe_geom* g, int n, int kk, int n_ids) {
  const long rows = long(n) * kk;
  // column blocks must tile the outputs; the pipeline runs 4 groups per trip
  // scales are read 8 groups (16 bytes) at a time
  if (g->inter % kGuCols || g->hidden % kDnCols || g->inter % 512 || g->hidden % 512) return false;
  return rows >= 1024 && rows >= 16L * n_ids;
}

int prefill_experts(const pmoe_geom* g, const uint8_t* slab, const uint16_t* x, int n, int kk,
                    const int32_t* order, const int4* tiles, const int32_t* n_tiles, int tile_m,
                    int max_tiles, uint16_t* h, void* y, int y_f32, hipStream_t st) {
  PMOE_REQUIRE(tile_m == 32 || tile_m == kTileM, "prefill: tile height must be 32 or 128");
  PMOE_REQUIRE(g->inter % 512 == 0 && g->hidden % 512 == 0,
               "prefill: hidden and inter must be multiples of 512");
  PMOE_REQUIRE(max_tiles > 0 && max_tiles <= (1 << 20), "prefill: tile count out of range");
  PMOE_REQUIRE(int64_t(n) * g->hidden < (int64_t(1) << 31) &&
                   int64_t(n) * kk * g->inter < (int64_t(1) << 31),
               "prefill: activations exceed 2^31 elements");
  const bool small = tile_m == 32;
  PrefillArgs a{};
  a.slab = slab;
  a.expert_bytes = g->expert_bytes;
  a.order = order;
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
    if (g->bits == 4 && small)
      gateup_mfma_kernel<4, 1><<<grid, kThreads, 0, st>>>(a);
    else if (g->bits == 4)
      gateup_mfma_kernel<4, kMB><<<grid, kThreads, 0, st>>>(a);
    else if (small)
      gateup_mfma_kernel<6, 1><<<grid, kThreads, 0, st>>>(a);
    else
      gateup_mfma_kernel<6, kMB><<<grid, kThreads, 0, st>>>(a);
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
  a.out_vec = (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  {
    const int items = g->hidden / kDnCols * max_tiles;
    dim3 grid((items + 7) / 8 * 8);
    ProfScope prof_scope(K_PREFILL_DOWN, st);
    if (g->bits == 4 && small)
      down_mfma_kernel<4, 1><<<grid, kThreads, 0, st>>>(a);
    else if (g->bits == 4)
      down_mfma_kernel<4, kMB><<<grid, kThreads, 0, st>>>(a);
    else if (small)
      down_mfma_kernel<6, 1><<<grid, kThreads, 0, st>>>(a);
    else
      down_mfma_kernel<6, kMB><<<grid, kThreads, 0, st>>>(a);
    PMOE_LAUNCH_CHECK("down_mfma_kernel");
  }
  return PMOE_OK;
}

}  // namespace pmoe
