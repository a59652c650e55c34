// Router logits tile: one wave computes TE x TN logits (experts x tokens)
// in the fixed fp32 summation order shared with the CPU oracle (bit for
// bit): element d = 512*t + 8*l + j is owned by lane l; each lane runs
// acc = fma(x_d, w_d, acc) for t ascending, j ascending (one 16-byte load of
// x and of w per t); the 64 lane partials are combined by an xor butterfly.
// Used by the plain router launch (router.hip) and by the decode router
// launch that also routes (decode.hip).
#pragma once

#include "pmoe_internal.h"

namespace pmoe {

constexpr int kRouterWaves = 4;  // waves per router block

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

// One stage of the 64-lane xor butterfly (distance D) over the C values a
// lane holds, C > 1: the two lanes of each pair add the same operands as
// wave_sum_bfly's v + xor_lane<D>(v), but each keeps only half of the values
// -- the lane whose bit D is 0 the first half, the other the second -- so
// the stage costs C / 2 exchanges instead of C.  Afterwards v[0, C / 2)
// holds the lane's half.  Distances 32 and 16 exchange with one
// v_permlane32_swap / v_permlane16_swap per pair of values (x's upper half
// or odd rows trade places with y's lower half or even rows).
template <int D, int C>
__device__ __forceinline__ void bfly_split(float (&v)[C]) {
  static_assert(C >= 2 && (C & (C - 1)) == 0, "a power of two of values");
  constexpr int H = C / 2;
  const bool hi = (threadIdx.x & D) != 0;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const uint32_t x = __float_as_uint(v[i]), y = __float_as_uint(v[i + H]);
    if constexpr (D == 32 || D == 16) {
      const auto r = D == 32 ? __builtin_amdgcn_permlane32_swap(x, y, false, false)
                             : __builtin_amdgcn_permlane16_swap(x, y, false, false);
      // low lanes: own x + partner's x; high lanes: partner's y + own y
      v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
      const float keep = hi ? v[i + H] : v[i];
      const float recv = xor_lane<D>(hi ? v[i] : v[i + H]);
      v[i] = keep + recv;
    }
  }
}

// The xor butterfly of wave_sum_bfly (distances 32, 16, 8, 4, 2, 1) over N
// values a lane holds, bit for bit the same sums: the first log2(N) stages
// split (bfly_split), the rest are whole.  Lane l ends with the sum of value
// index lane_value_index<N>(l) in v[0].
template <int N>
__device__ __forceinline__ void wave_sum_split(float (&v)[N]) {
  if constexpr (N >= 2) bfly_split<32, N>(v);
  if constexpr (N >= 4) bfly_split<16, N / 2>(*reinterpret_cast<float(*)[N / 2]>(&v[0]));
  if constexpr (N >= 8) bfly_split<8, N / 4>(*reinterpret_cast<float(*)[N / 4]>(&v[0]));
  if constexpr (N >= 16) bfly_split<4, N / 8>(*reinterpret_cast<float(*)[N / 8]>(&v[0]));
  if constexpr (N >= 32) bfly_split<2, N / 16>(*reinterpret_cast<float(*)[N / 16]>(&v[0]));
  static_assert(N <= 32, "at most 32 values");
  if constexpr (N < 2) v[0] = v[0] + xor_lane<32>(v[0]);
  if constexpr (N < 4) v[0] = v[0] + xor_lane<16>(v[0]);
  if constexpr (N < 8) v[0] = v[0] + xor_lane<8>(v[0]);
  if constexpr (N < 16) v[0] = v[0] + xor_lane<4>(v[0]);
  if constexpr (N < 32) v[0] = v[0] + xor_lane<2>(v[0]);
  v[0] = v[0] + xor_lane<1>(v[0]);
}

// Which of the N values lane l holds after wave_sum_split: the split
// stages' lane bits, distance 32 (worth N / 2) down.
template <int N>
__device__ __forceinline__ int split_index(int l) {
  int idx = 0;
  int h = N / 2;
#pragma unroll
  for (int d = 32; d >= 1 && h >= 1; d >>= 1, h >>= 1)
    if (l & d) idx += h;
  return idx;
}

// Logits of experts [e0, e0 + TE) x tokens [n0, n0 + TN) by the calling wave
// (e0 < e).  Rows e < n_w come from w (+ bias), row n_w (if e > n_w) from
// w_extra; out has ld = e columns.  Passes of 512 columns are loaded UNR at
// a time (one memory round trip per group: compiled per pass, a wave waited
// for one pass's loads before issuing the next pass's); FULL (d a multiple
// of 512) drops the column guard.  DEV stores at device scope (written
// through to where every XCD reads it), for a reader in the same launch.
template <int TE, int TN, int UNR, bool FULL, bool DEV>
__device__ __forceinline__ void router_tile(const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ w,
                                            const uint16_t* __restrict__ w_extra,
                                            const float* __restrict__ bias, int n, int d, int e,
                                            int n_w, float* __restrict__ out, int e0, int n0) {
  const int lane = threadIdx.x & 63;
  float acc[TE][TN];
#pragma unroll
  for (int i = 0; i < TE; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;

  // UNR passes at a time: every load of the group is issued before the
  // first FMA (sched_barrier keeps the compiler from sinking them), then the
  // FMAs run in pass order.  Passes past the end and columns past d load an
  // in-bounds address and skip their FMAs.
  const int passes = (d + 511) / 512;
  for (int t0 = 0; t0 < passes; t0 += UNR) {
    uint4 wv[UNR][TE], xv[UNR][TN];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int col = min(min(t0 + u, passes - 1) * 512 + lane * 8, d - 8);
#pragma unroll
      for (int i = 0; i < TE; ++i) {
        const int ei = min(e0 + i, e - 1);
        const uint16_t* src = ei < n_w ? w + size_t(ei) * d : w_extra;
        wv[u][i] = *reinterpret_cast<const uint4*>(src + col);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int nj = min(n0 + j, n - 1);
        xv[u][j] = *reinterpret_cast<const uint4*>(x + size_t(nj) * d + col);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int col = (t0 + u) * 512 + lane * 8;
      if (t0 + u < passes && (FULL || col < d)) {
#pragma unroll
        for (int i = 0; i < TE; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) fma8(acc[i][j], xv[u][j], wv[u][i]);
      }
    }
  }
  // the TE x TN sums, split over the lanes: lane l ends with logit
  // split_index(l) (lanes that differ only below the split bits hold the
  // same one; the lowest of them stores it)
  constexpr int N = TE * TN;
  float v[N];
#pragma unroll
  for (int i = 0; i < TE; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) v[i * TN + j] = acc[i][j];
  wave_sum_split<N>(v);
  constexpr int kLow = 64 / N - 1;  // lane bits below the split ones
  const int idx = split_index<N>(lane);
  const int i = idx / TN, j = idx - (idx / TN) * TN;
  if ((lane & kLow) == 0 && e0 + i < e && n0 + j < n) {
    const bool biased = bias && e0 + i < n_w;
    float* o = out + size_t(n0 + j) * e + e0 + i;
    const float s = v[0];
    const float r = biased ? s + bias[e0 + i] : s;
    if (DEV)
      __hip_atomic_store(o, r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      *o = r;
  }
}

}  // namespace pmoe
