// Grouped dequant-GEMV primitives shared by the decode kernels (decode.hip,
// decode_fused.hip).
//
// Per lane and unit (a whole or half quantization group): the packed weight
// words arrive as 16-byte loads, each 32-bit word is turned into bf16 pairs
// (128+q) with one and/or (4-bit) or a funnel shift (6-bit), and
// v_dot2_f32_bf16 accumulates x*(128+q) in fp32.  With xs = sum of the
// unit's x and (s, b) its group's scale and bias, the unit's contribution is
//   s*sum(x*q) + b*xs = s*acc + (b - 128*s)*xs,
// so dequantised weights are never materialised.  Rows are reduced across
// their LPR lanes with an xor butterfly.
#pragma once

#include "pmoe_internal.h"
#include "pmoe_kernels.h"

// Tuning knobs (compile-time): rows per wave step override (0 = sized from
// the register budget), non-temporal weight loads, minimum waves per SIMD.
#ifndef PMOE_FORCE_R
#define PMOE_FORCE_R 0
#endif
#ifndef PMOE_NT_LOADS
#define PMOE_NT_LOADS 1
#endif
#ifndef PMOE_MIN_WAVES
#define PMOE_MIN_WAVES 3
#endif
#ifndef PMOE_AND_OR
#define PMOE_AND_OR 1
#endif

namespace pmoe {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), c, false);
}

// A lane's share of a weight row is made of units of UB packed bytes:
//   UB = 32: a whole 4-bit quantization group (64 values);
//   UB = 16: half of a 4-bit group (32 values).  Lane sub of a row owns
//            units sub + LPR*j, so load instruction j covers the contiguous
//            16*LPR bytes [16*LPR*j, 16*LPR*(j+1)) of the row;
//   UB = 48: a whole 6-bit group (6-bit fields straddle 16-byte chunks).
template <int UB>
struct Unit {
  static_assert(UB == 16 || UB == 32 || UB == 48, "unit of 16, 32 or 48 bytes");
  static constexpr int kBits = UB == 48 ? 6 : 4;
  static constexpr int kVals = UB * 8 / kBits;  // 32, 64, 64
  static constexpr int kWords = UB / 4;         // 4, 8, 12
};

// Activations of one unit, pre-arranged as the bf16 pairs the weight words
// of that unit are unpacked into, plus the unit's sum.
template <int UB>
struct GroupAct {
  uint32_t p[Unit<UB>::kVals / 2];
  float sum;
};

// 16 bytes of activations; COHERENT reads at device scope (data written by
// other blocks of the same launch) as two 8-byte atomic loads.
template <bool COHERENT>
__device__ __forceinline__ uint4 load_act16(const uint4* p) {
  if (!COHERENT) return *p;
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4(uint32_t(lo), uint32_t(lo >> 32), uint32_t(hi), uint32_t(hi >> 32));
}

// Load one unit of activations starting at src (16-byte aligned) into pair
// order.
template <int UB, bool COHERENT = false>
__device__ __forceinline__ void load_group_act(const uint16_t* src, GroupAct<UB>& a) {
  const uint4* v = reinterpret_cast<const uint4*>(src);
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < Unit<UB>::kVals / 8; ++c) {
    const uint4 d = load_act16<COHERENT>(v + c);
    // the unit's sum as dot products of the bf16 pairs with (1, 1)
    constexpr uint32_t kOnes = 0x3F803F80u;
    s = dot2(d.w, kOnes, dot2(d.z, kOnes, dot2(d.y, kOnes, dot2(d.x, kOnes, s))));
    if (Unit<UB>::kBits == 4) {
      // word c of the unit holds values 8c..8c+7; pair i is (x_{8c+i}, x_{8c+i+4})
      a.p[4 * c + 0] = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
      a.p[4 * c + 1] = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
      a.p[4 * c + 2] = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
      a.p[4 * c + 3] = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
    } else {
      // pair p is (x_{2p}, x_{2p+1}): the natural bf16 pairs
      a.p[4 * c + 0] = d.x;
      a.p[4 * c + 1] = d.y;
      a.p[4 * c + 2] = d.z;
      a.p[4 * c + 3] = d.w;
    }
  }
  a.sum = s;
}

template <int UB>
struct GroupW {
  static constexpr int kWords = Unit<UB>::kWords;
  uint32_t w[kWords];
  uint32_t sb;  // the group's bf16 scale (low half) and bias (high half)
  __device__ __forceinline__ float s() const { return __uint_as_float(sb << 16); }
  __device__ __forceinline__ float b() const { return __uint_as_float(sb & 0xFFFF0000u); }
};

// Unit u of a row: its packed words and its group's scale and bias.
template <int UB>
__device__ __forceinline__ void load_group_w(const uint32_t* wrow, const uint16_t* srow,
                                             const uint16_t* brow, int u, GroupW<UB>& q) {
  constexpr int kWords = GroupW<UB>::kWords;
  const u32x4* v = reinterpret_cast<const u32x4*>(wrow + size_t(u) * kWords);
#pragma unroll
  for (int c = 0; c < kWords / 4; ++c) {
    // Non-temporal only for 16-byte units, where one load instruction covers
    // whole contiguous lines of the row.  With 32- or 48-byte units two or
    // three instructions share each line, and a normal load keeps the line
    // in L2 for the next one (6-bit Qwen3-Next-shaped verify step: 119 ->
    // 108 us).
    u32x4 d;
    if (PMOE_NT_LOADS && UB == 16)
      d = __builtin_nontemporal_load(v + c);
    else
      d = v[c];
    q.w[4 * c + 0] = d.x;
    q.w[4 * c + 1] = d.y;
    q.w[4 * c + 2] = d.z;
    q.w[4 * c + 3] = d.w;
  }
  const int g = u * Unit<UB>::kVals / 64;
  q.sb = uint32_t(srow[g]) | (uint32_t(brow[g]) << 16);
}

// (v & mask) | bias in one v_and_or_b32.  A VOP3 instruction takes no
// literal operand on this target, so written plainly the compiler emits a
// separate and + or pair (two VOP2 with literals); here the mask comes from an
// SGPR and the OR constant from a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t bias) {
#if PMOE_AND_OR
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(bias));
  return r;
#else
  return (v & mask) | bias;
#endif
}

// bf16 (128+q) pairs (q_i, q_{i+4}) of the 4-bit word w: pair k holds the
// nibbles at bits 4k and 16+4k
template <int K>
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, uint32_t k43) {
  return and_or(K ? w >> (4 * K) : w, 0x000F000Fu, k43);
}

// sum over the unit of x*(128+q)
template <int UB>
__device__ __forceinline__ float group_dot(const GroupW<UB>& q, const GroupAct<UB>& a) {
  float acc = 0.0f;
  if (Unit<UB>::kBits == 4) {
    // the OR constant, held in a VGPR for and_or (a pure asm: one register
    // shared by every unit)
    uint32_t k43;
#if PMOE_AND_OR
    asm("v_mov_b32 %0, 0x43004300" : "=v"(k43));
#else
    k43 = 0x43004300u;
#endif
#pragma unroll
    for (int c = 0; c < Unit<UB>::kWords; ++c) {
      const uint32_t w = q.w[c];
      acc = dot2(a.p[4 * c + 0], nib_pair<0>(w, k43), acc);
      acc = dot2(a.p[4 * c + 1], nib_pair<1>(w, k43), acc);
      acc = dot2(a.p[4 * c + 2], nib_pair<2>(w, k43), acc);
      acc = dot2(a.p[4 * c + 3], nib_pair<3>(w, k43), acc);
    }
  } else {
    uint32_t k43;
#if PMOE_AND_OR
    asm("v_mov_b32 %0, 0x43004300" : "=v"(k43));
#else
    k43 = 0x43004300u;
#endif
#pragma unroll
    for (int p = 0; p < 32; ++p) {
      const int bit = 12 * p;
      const int wi = bit >> 5, sh = bit & 31;
      uint32_t f;
      if (sh + 12 <= 32)
        f = q.w[wi] >> sh;
      else
        f = __builtin_amdgcn_alignbit(q.w[wi + 1], q.w[wi], sh);
      // (f & 0x3F) | ((f << 10) & 0x3F0000) | 0x43004300 as two and_or (the
      // inner result has bits 0-5 clear)
      const uint32_t pr = and_or(f, 0x3Fu, and_or(f << 10, 0x003F0000u, k43));
      acc = dot2(a.p[p], pr, acc);
    }
  }
  return acc;
}

__device__ __forceinline__ float group_term(float acc, float s, float b, float xs, float part) {
  return __builtin_fmaf(s, acc, __builtin_fmaf(b - 128.0f * s, xs, part));
}

// ---------------------------------------------------------------- GEMV core
//
// A wave computes rows o = wrow0 + st*RPW + rsub (st < R, RPW = 64/LPR rows
// per step, lane = rsub*LPR + sub) of one expert's projection(s): each lane
// owns units sub + LPR*j (j < GPL) of its row (past the row's last unit a
// lane re-loads that unit and leaves it out of the sum).  The weights of all R steps
// (one or two projections) are held in registers (GemvRegs) and reused for
// every activation row of the expert.

template <int UB, int LPR, int GPL, int R, bool DUAL>
struct GemvRegs {
  GroupW<UB> q0[R][GPL];
  GroupW<UB> q1[DUAL ? R : 1][DUAL ? GPL : 1];
};

// Issue the whole weight burst of the wave (R steps x GPL units x 1-2
// projections) for the expert in `slot`.  Rows past rows_out re-load the
// last row (in bounds, never stored).
template <int UB, int LPR, int GPL, int R, bool DUAL>
__device__ __forceinline__ void gemv_load(const GemvArgs& a, int slot, int wrow0,
                                          GemvRegs<UB, LPR, GPL, R, DUAL>& q) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPR;
  const int rsub = lane / LPR;
  const int units = a.cols / Unit<UB>::kVals;
  const int groups = a.cols / 64;
  const int wpr = a.cols * Unit<UB>::kBits / 32;
  const uint8_t* base = a.slab + size_t(slot) * a.expert_bytes;
  const uint32_t* W0 = reinterpret_cast<const uint32_t*>(base + a.p0.w);
  const uint16_t* S0 = reinterpret_cast<const uint16_t*>(base + a.p0.s);
  const uint16_t* B0 = reinterpret_cast<const uint16_t*>(base + a.p0.b);
  const uint32_t* W1 = reinterpret_cast<const uint32_t*>(base + a.p1.w);
  const uint16_t* S1 = reinterpret_cast<const uint16_t*>(base + a.p1.s);
  const uint16_t* B1 = reinterpret_cast<const uint16_t*>(base + a.p1.b);
#pragma unroll
  for (int st = 0; st < R; ++st) {
    const int o = min(wrow0 + st * RPW + rsub, a.rows_out - 1);
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      const int u = min(sub + LPR * j, units - 1);
      load_group_w<UB>(W0 + size_t(o) * wpr, S0 + size_t(o) * groups, B0 + size_t(o) * groups,
                       u, q.q0[st][j]);
      if (DUAL)
        load_group_w<UB>(W1 + size_t(o) * wpr, S1 + size_t(o) * groups,
                         B1 + size_t(o) * groups, u, q.q1[DUAL ? st : 0][DUAL ? j : 0]);
    }
  }
}

// The lane's activation units of one activation row (cols values).
template <int UB, int LPR, int GPL, bool COHERENT = false>
__device__ __forceinline__ void gemv_load_act(const uint16_t* src, int cols,
                                              GroupAct<UB> (&act)[GPL]) {
  const int sub = (threadIdx.x & 63) % LPR;
  const int units = cols / Unit<UB>::kVals;
#pragma unroll
  for (int j = 0; j < GPL; ++j) {
    const int u = min(sub + LPR * j, units - 1);
    load_group_act<UB, COHERENT>(src + size_t(u) * Unit<UB>::kVals, act[j]);
  }
}

// Outputs of the R steps for the activation row held in act; store(st, o,
// value) receives each finished row output (value = silu(g)*u for DUAL):
// from the row group's first lane, for rows below rows_out, or (ALL) from
// every lane of the row group, every row, unmasked.
template <int UB, int LPR, int GPL, int R, bool DUAL, class Store, bool ALL = false>
__device__ __forceinline__ void gemv_rows(const GemvArgs& a,
                                          GemvRegs<UB, LPR, GPL, R, DUAL>& q,
                                          const GroupAct<UB> (&act)[GPL], int wrow0,
                                          Store store) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPR;
  const int rsub = lane / LPR;
  const int units = a.cols / Unit<UB>::kVals;
#pragma unroll
  for (int st = 0; st < R; ++st) {
    // Opaque to the optimiser: without this the unpacked pairs of every
    // row are hoisted out of the row loop and spill.
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
#pragma unroll
      for (int c = 0; c < GroupW<UB>::kWords; ++c) {
        asm volatile("" : "+v"(q.q0[st][j].w[c]));
        if (DUAL) asm volatile("" : "+v"(q.q1[DUAL ? st : 0][DUAL ? j : 0].w[c]));
      }
    }
    float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      if (sub + LPR * j < units) {
        p0 = group_term(group_dot<UB>(q.q0[st][j], act[j]), q.q0[st][j].s(), q.q0[st][j].b(),
                        act[j].sum, p0);
        if (DUAL) {
          const GroupW<UB>& w1 = q.q1[DUAL ? st : 0][DUAL ? j : 0];
          p1 = group_term(group_dot<UB>(w1, act[j]), w1.s(), w1.b(), act[j].sum, p1);
        }
      }
    }
    float v = group_sum<LPR>(p0);
    if (DUAL) v = silu_fast(v) * group_sum<LPR>(p1);
    const int o = wrow0 + st * RPW + rsub;
    if (ALL || (sub == 0 && o < a.rows_out)) store(st, o, v);
  }
}

// One expert's projection(s) for its activation rows rlist[0..m_total).
// Activations of the first row are requested first (L2 hits), then the whole
// weight burst of the wave; vector loads retire in order, so row 0 starts as
// soon as its own words have landed.  store(t_row, st, o, value).
template <int UB, int LPR, int GPL, int R, bool DUAL, class Act, class Store>
__device__ __forceinline__ void gemv_expert(const GemvArgs& a, int slot, int m_total,
                                            const int32_t* rlist, int wrow0, Act act_row,
                                            Store store) {
  GroupAct<UB> act[GPL];
  int r = rlist[0];
  gemv_load_act<UB, LPR, GPL>(act_row(r), a.cols, act);
  __builtin_amdgcn_sched_barrier(0);
  GemvRegs<UB, LPR, GPL, R, DUAL> q;
  gemv_load<UB, LPR, GPL, R, DUAL>(a, slot, wrow0, q);
  __builtin_amdgcn_sched_barrier(0);
  for (int m = 0; m < m_total; ++m) {
    if (m > 0) {
      r = rlist[m];
      gemv_load_act<UB, LPR, GPL>(act_row(r), a.cols, act);
      __builtin_amdgcn_sched_barrier(0);
    }
    gemv_rows<UB, LPR, GPL, R, DUAL>(a, q, act, wrow0,
                                       [&](int st, int o, float v) { store(r, st, o, v); });
  }
}

struct Shape {
  int lpr, gpl, ub;  // lanes per row, units per lane, unit bytes
};

// Row shape for rows of `cols` values.
// 4-bit rows of >= 64 groups: whole groups (32-byte units) on 64 lanes, the
// last step masked when the count is not a multiple of 64 -- the most bytes
// in flight per register, for launches whose waves are all resident at once
// -- or, with half_groups, 16-byte units on 64 lanes, each load instruction
// covering a contiguous 1 KB of the row (the faster pattern once waves
// queue behind each other).  Shorter 4-bit rows: half groups on the largest
// power of two of lanes dividing the unit count when that leaves at most 3
// units per lane, so every lane has work; else one unit per lane (64 lanes at
// most), masked.
// 6-bit (48-byte group units): the smallest power of two >= groups (8..64).
inline Shape pick_shape(int bits, int cols, bool half_groups = false) {
  if (cols <= 0 || cols % 64 || cols > 8192 || (bits != 4 && bits != 6)) return {0, 0, 0};
  const int groups = cols / 64;
  if (bits == 4 && groups >= 64)
    return half_groups ? Shape{64, (2 * groups + 63) / 64, 16} : Shape{64, (groups + 63) / 64, 32};
  const int units = bits == 4 ? 2 * groups : groups;
  const int ub = bits == 4 ? 16 : 48;
  if (bits == 4 && units % 8 == 0) {
    int lpr = 64;
    while (units % lpr) lpr >>= 1;
    if (units / lpr <= 3) return {lpr, units / lpr, ub};
  }
  int lpr = 8;
  while (lpr < units && lpr < 64) lpr <<= 1;
  return {lpr, (units + lpr - 1) / lpr, ub};
}

// Gate/up row shape of the decode launches (both decode paths use it, so
// they stay bit-identical): half-group units (each load instruction a
// contiguous 1 KB of the row) for rows of up to 2 units per lane, whole
// groups above that, where 4 half-group units per lane exceed the register
// budget (decode.hip).
Shape gateup_shape(int bits, const GemvArgs& gu, int max_experts);

}  // namespace pmoe
