// Block-level routing helpers shared by the decode kernels.
//
// Every block of a decode GEMV launch recomputes the layer's routing from the
// fp32 router logits (a few hundred floats) instead of waiting for a separate
// routing launch.  The computation is deterministic and uses only separately
// rounded float ops, so every block, and the CPU oracle, get identical bits:
//   * top-k per token: radix select on order-preserving keys with wave
//     ballots, ties to the lower expert id, picks sorted by (value desc, id
//     asc) -- softmax(+renorm) or sigmoid+bias with grouped selection and
//     routed scaling (tests/test_stream.py:191-196; streaming.py:2424-2442);
//   * active experts: a bitmap of the used ids, listed in ascending order;
//   * rows of an expert: the flat (token, slot) rows holding its id, in
//     ascending order -- the stable dispatch of streaming.py:794.
#pragma once

#include "pmoe_internal.h"

namespace pmoe {

constexpr int kRouteMaxK = 16;
constexpr int kRouteMaxRows = 256;   // n * kk per decode launch
constexpr int kRouteMaxIds = 1024;   // E + shared
constexpr int kRouteMaxSigE = 512;   // sigmoid scoring: experts per token

struct RouteDev {
  const float* logits;  // [n, ld]; column e (when ld > e) is the shared gate
  int ld;
  const float* bias;    // [e] (sigmoid scoring)
  int scoring, n, e, k, kk, norm, n_group, topk_group;
  float scale;
  int shared_gate;      // shared weight = sigmoid(logits[n, e]) instead of 1
};

struct WaveTmp {
  float tv[kRouteMaxK], tx[kRouteMaxK], ov[kRouteMaxK], ox[kRouteMaxK];
  int ti[kRouteMaxK], oi[kRouteMaxK];
  float c[kRouteMaxSigE];
};

struct RouteLds {
  int32_t ids[kRouteMaxRows];     // flat row -> expert id (shared: e)
  float w[kRouteMaxRows];         // flat row -> combine weight
  uint64_t bits[kRouteMaxIds / 64];
  int32_t active[kRouteMaxIds];
  int32_t n_active;
};

__device__ __forceinline__ uint32_t order_key(float v) {
  if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal: one key
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0));
}

// Lanes of the wave where c holds (one compare into an SGPR pair).
__device__ __forceinline__ uint64_t wave_ballot(bool c) { return __builtin_amdgcn_ballot_w64(c); }

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Top-k of per-lane values v[i] (id lane + 64*i, valid when id < n_valid).
// Writes the k picks sorted by (value desc, id asc) to out_v/out_i and, when
// EXTRA, carries extra[i] along to out_x.  tmp_* hold k entries.
template <bool EXTRA, int EPL>
__device__ __forceinline__ void wave_topk_radix(const float (&v)[EPL], int n_valid, int k,
                                                float* out_v, int* out_i,
                                                const float (&extra)[EPL], float* out_x,
                                                float* tmp_v, int* tmp_i, float* tmp_x) {
  const int lane = threadIdx.x & 63;
  uint32_t key[EPL];
  bool valid[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    valid[i] = lane + 64 * i < n_valid;
    key[i] = valid[i] ? order_key(v[i]) : 0u;
  }
  // p = the k-th largest key: the largest value whose count of keys >= p is
  // at least k, found two bits per step (three candidate thresholds).
  // Invalid entries hold key 0, below every candidate (all are >= 1).
  uint32_t p = 0;
  for (int b = 30; b >= 0; b -= 2) {
    const uint32_t c1 = p | (1u << b), c2 = p | (2u << b), c3 = p | (3u << b);
    int n1 = 0, n2 = 0, n3 = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      n1 += __popcll(wave_ballot(key[i] >= c1));
      n2 += __popcll(wave_ballot(key[i] >= c2));
      n3 += __popcll(wave_ballot(key[i] >= c3));
    }
    p = n3 >= k ? c3 : (n2 >= k ? c2 : (n1 >= k ? c1 : p));
  }
  int gt = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) gt += __popcll(wave_ballot(key[i] > p));
  const int need = k - gt;
  int run_eq = 0, run_sel = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const bool eq = valid[i] && key[i] == p;
    const uint64_t eqm = wave_ballot(eq);
    const bool sel = (valid[i] && key[i] > p) || (eq && run_eq + lanes_below(eqm) < need);
    run_eq += __popcll(eqm);
    const uint64_t selm = wave_ballot(sel);
    if (sel) {
      const int pos = run_sel + lanes_below(selm);
      tmp_v[pos] = v[i];
      tmp_i[pos] = lane + 64 * i;
      if (EXTRA) tmp_x[pos] = extra[i];
    }
    run_sel += __popcll(selm);
  }
  wave_lds_sync();
  if (lane < k) {
    const float mv = tmp_v[lane];
    const int mi = tmp_i[lane];
    float ovs[kRouteMaxK];
    int ois[kRouteMaxK];
#pragma unroll
    for (int j = 0; j < kRouteMaxK; ++j) {  // all loads in flight at once
      if (j < k) {
        ovs[j] = tmp_v[j];
        ois[j] = tmp_i[j];
      }
    }
    int rank = 0;
#pragma unroll
    for (int j = 0; j < kRouteMaxK; ++j)
      if (j < k) rank += (ovs[j] > mv || (ovs[j] == mv && ois[j] < mi)) ? 1 : 0;
    out_v[rank] = mv;
    out_i[rank] = mi;
    if (EXTRA) out_x[rank] = tmp_x[lane];
  }
  wave_lds_sync();
}

// Logit loads: COHERENT reads the logits at device scope (they were written
// by other blocks of the same launch and may be stale in this XCD's L2).
template <bool COHERENT>
__device__ __forceinline__ float load_logit(const float* p) {
  if (COHERENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}

// Route token t with the calling wave: writes L.ids / L.w for its kk rows
// and, when inds_out is set, the routing outputs [n, k].
template <int EPL, bool COHERENT = false>
__device__ void route_token(const RouteDev& r, int t, RouteLds& L, WaveTmp& W, int32_t* inds_out,
                            float* w_out) {
  const int lane = threadIdx.x & 63;
  const int e = r.e, k = r.k;
  const float* row = r.logits + size_t(t) * r.ld;
  float v[EPL], x[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int ei = lane + 64 * i;
    v[i] = ei < e ? load_logit<COHERENT>(row + ei) : 0.0f;
    x[i] = 0.0f;
  }
  float wk = 0.0f;
  int ik = 0;
  if (r.scoring == PMOE_SCORE_SOFTMAX) {
    wave_topk_radix<false, EPL>(v, e, k, W.ov, W.oi, x, nullptr, W.tv, W.ti, W.tx);
    const float m = W.ov[0];
    // lane j < k holds exp(v_j - m); the sum runs in pick order j = 0..k-1
    const float ej = lane < k ? pexp(W.ov[lane] - m) : 0.0f;
    float s = 0.0f;
    if (r.norm) {
      for (int j = 0; j < k; ++j) s = s + __shfl(ej, j, kWave);
    } else {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (lane + 64 * i < e) acc = acc + pexp(v[i] - m);
      s = wave_sum_bfly(acc);
    }
    if (lane < k) {
      ik = W.oi[lane];
      wk = ej / s;
    }
  } else {
    float c[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int ei = lane + 64 * i;
      if (ei < e) {
        x[i] = psigmoid(v[i]);
        c[i] = x[i] + r.bias[ei];
        W.c[ei] = c[i];
      } else {
        c[i] = 0.0f;
      }
    }
    wave_lds_sync();
    if (r.n_group > 1) {
      const int gs = e / r.n_group;
      float gscore[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) gscore[i] = 0.0f;
      if (lane < r.n_group) {
        float t1 = -__builtin_inff(), t2 = -__builtin_inff();
        for (int j = 0; j < gs; ++j) {
          const float xv = W.c[lane * gs + j];
          if (xv > t1) {
            t2 = t1;
            t1 = xv;
          } else if (xv > t2) {
            t2 = xv;
          }
        }
        gscore[0] = t1 + t2;
      }
      // group picks land in the upper half of ov/oi (topk_group <= 8)
      wave_topk_radix<false, EPL>(gscore, r.n_group, r.topk_group, W.ov + 8, W.oi + 8, x,
                                  nullptr, W.tv, W.ti, W.tx);
      uint64_t keep = 0;
      for (int j = 0; j < r.topk_group; ++j) keep |= 1ull << W.oi[8 + j];
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int ei = lane + 64 * i;
        if (ei < e && !((keep >> (ei / gs)) & 1ull)) c[i] = 0.0f;
      }
    }
    wave_topk_radix<true, EPL>(c, e, k, W.ov, W.oi, x, W.ox, W.tv, W.ti, W.tx);
    float s = 0.0f;
    for (int j = 0; j < k; ++j) s = s + W.ox[j];
    if (lane < k) {
      float w = W.ox[lane];
      if (r.norm) w = w / s;
      wk = w * r.scale;
      ik = W.oi[lane];
    }
  }
  if (lane < k) {
    L.ids[t * r.kk + lane] = ik;
    L.w[t * r.kk + lane] = wk;
    if (inds_out) {
      inds_out[size_t(t) * k + lane] = ik;
      w_out[size_t(t) * k + lane] = wk;
    }
  }
  if (r.kk > k && lane == 0) {
    L.ids[t * r.kk + k] = e;  // shared expert column
    L.w[t * r.kk + k] = r.shared_gate ? psigmoid(load_logit<COHERENT>(row + e)) : 1.0f;
  }
}

// Route all tokens (waves take tokens round robin), then list the active
// experts in ascending id order.  Ends with a block barrier.
template <int EPL, int NW, bool COHERENT = false>
__device__ void route_block(const RouteDev& r, RouteLds& L, WaveTmp* W, int32_t* inds_out,
                            float* w_out) {
  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int n_ids = r.e + (r.kk > r.k ? 1 : 0);
  for (int i = tid; i < kRouteMaxIds / 64; i += NW * 64) L.bits[i] = 0;
  for (int t = wv; t < r.n; t += NW)
    route_token<EPL, COHERENT>(r, t, L, W[wv], inds_out, w_out);
  __syncthreads();
  const int rows = r.n * r.kk;
  for (int i = tid; i < rows; i += NW * 64) {
    const int id = L.ids[i];
    atomicOr(reinterpret_cast<unsigned long long*>(&L.bits[id >> 6]), 1ull << (id & 63));
  }
  __syncthreads();
  if (wv == 0) {
    const int lane = tid & 63;
    int base = 0;
    for (int wd = 0; wd < (n_ids + 63) / 64; ++wd) {
      const uint64_t b = L.bits[wd];
      const bool mine = (b >> lane) & 1ull;
      if (mine) L.active[base + lanes_below(b)] = wd * 64 + lane;
      base += __popcll(b);
    }
    if (lane == 0) L.n_active = base;
  }
  __syncthreads();
}

// Routing record in global memory: what block (0, 0) of the gate/up launch
// publishes for the down launch (same layout as the LDS copy).
struct RouteRecord {
  int32_t ids[kRouteMaxRows];
  float w[kRouteMaxRows];
  int32_t active[kRouteMaxIds];
  int32_t n_active;
};

__device__ __forceinline__ void publish_route(const RouteLds& L, int rows, int n_ids,
                                              RouteRecord* g) {
  for (int i = threadIdx.x; i < rows; i += blockDim.x) {
    g->ids[i] = L.ids[i];
    g->w[i] = L.w[i];
  }
  for (int i = threadIdx.x; i < n_ids; i += blockDim.x) g->active[i] = L.active[i];
  if (threadIdx.x == 0) g->n_active = L.n_active;
}

__device__ __forceinline__ void load_route(const RouteRecord* g, int rows, int n_ids, RouteLds& L) {
  for (int i = threadIdx.x; i < rows; i += blockDim.x) {
    L.ids[i] = g->ids[i];
    L.w[i] = g->w[i];
  }
  for (int i = threadIdx.x; i < n_ids; i += blockDim.x) L.active[i] = g->active[i];
  if (threadIdx.x == 0) L.n_active = g->n_active;
  __syncthreads();
}

// Rows (ascending) whose id is `id`, gathered by one wave into out[]; returns
// their count.
__device__ __forceinline__ int wave_rows_of(const RouteLds& L, int rows, int id, int32_t* out) {
  const int lane = threadIdx.x & 63;
  int m = 0;
  for (int base = 0; base < rows; base += 64) {
    const int r = base + lane;
    const bool hit = r < rows && L.ids[r] == id;
    const uint64_t mask = wave_ballot(hit);
    if (hit) out[m + lanes_below(mask)] = r;
    m += __popcll(mask);
  }
  wave_lds_sync();
  return m;
}

}  // namespace pmoe
