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
#pragma unroll
  for (int i = 0; i < TE; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const float s = wave_sum_bfly(acc[i][j]);
      if (lane == ((i * TN + j) & 63) && e0 + i < e && n0 + j < n) {
        const bool biased = bias && e0 + i < n_w;
        float* o = out + size_t(n0 + j) * e + e0 + i;
        const float v = biased ? s + bias[e0 + i] : s;
        if (DEV)
          __hip_atomic_store(o, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          *o = v;
      }
    }
}

}  // namespace pmoe
