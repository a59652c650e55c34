// Decode-sized routing + dispatch in one launch.
//
// Given fp32 router logits for n <= 64 tokens, one 1024-thread block
//   1. selects each token's top-k (one wave per token) and its weights,
//      with the same semantics and bit-exact results as route_softmax_kernel /
//      route_sigmoid_kernel (router.hip), and
//   2. groups the n*kk flat (token, slot) rows by expert exactly like the
//      stable dispatch in dispatch.hip (ids never leave LDS), and
//   3. zeroes the arrival counters the fused combine of the down projection
//      uses later on the same stream.
// Replaces, for decode, the block's top-k (tests/test_stream.py:191-196,
// streaming.py:2424-2442) and the argsort dispatch (streaming.py:789-808).
//
// Top-k by radix select: floats map to order-preserving u32 keys; the k-th
// largest key is found one bit at a time with wave ballots (32 steps, no
// cross-lane data movement), then ties at that key go to the lowest expert
// ids, and the k picks are ranked by (value desc, id asc).
#include "pmoe_internal.h"
#include "pmoe_kernels.h"

namespace pmoe {

namespace {

constexpr int kMaxK = 16;
constexpr int kMaxTokens = 64;
constexpr int kMaxRows = 1024;
constexpr int kMaxIds = 1024;

__device__ __forceinline__ uint32_t order_key(float v) {
  if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal: one key
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0));
}

// Top-k of per-lane values v[i] (id lane + 64*i, valid when id < n_valid).
// Writes the k picks sorted by (value desc, id asc) to out_v/out_i (LDS,
// k entries) and, when EXTRA, carries extra[i] along to out_x.
template <bool EXTRA, int EPL>
__device__ __forceinline__ void wave_topk_radix(const float (&v)[EPL], int epl, int n_valid, int k,
                                                float* out_v, int* out_i, const float (&extra)[EPL],
                                                float* out_x, float* tmp_v, int* tmp_i,
                                                float* tmp_x) {
  const int lane = threadIdx.x & 63;
  uint32_t key[EPL];
  bool valid[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    valid[i] = i < epl && lane + 64 * i < n_valid;
    key[i] = valid[i] ? order_key(v[i]) : 0u;
  }
  uint32_t p = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = p | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (i < epl) cnt += __popcll(__ballot(valid[i] && key[i] >= cand));
    if (cnt >= k) p = cand;
  }
  int gt = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (i < epl) gt += __popcll(__ballot(valid[i] && key[i] > p));
  const int need = k - gt;
  int run_eq = 0, run_sel = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    if (i < epl) {
      const bool eq = valid[i] && key[i] == p;
      const uint64_t eqm = __ballot(eq);
      const bool sel = (valid[i] && key[i] > p) || (eq && run_eq + lanes_below(eqm) < need);
      run_eq += __popcll(eqm);
      const uint64_t selm = __ballot(sel);
      if (sel) {
        const int pos = run_sel + lanes_below(selm);
        tmp_v[pos] = v[i];
        tmp_i[pos] = lane + 64 * i;
        if (EXTRA) tmp_x[pos] = extra[i];
      }
      run_sel += __popcll(selm);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < k) {
    const float mv = tmp_v[lane];
    const int mi = tmp_i[lane];
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      const float ov = tmp_v[j];
      const int oi = tmp_i[j];
      rank += (ov > mv || (ov == mv && oi < mi)) ? 1 : 0;
    }
    out_v[rank] = mv;
    out_i[rank] = mi;
    if (EXTRA) out_x[rank] = tmp_x[lane];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct RouteDecodeArgs {
  const float* logits;   // [n, E]
  const float* bias;     // [E] (sigmoid scoring)
  int n, e, k, kk, norm, n_group, topk_group;
  float scale;
  int scoring;
  int32_t* inds;         // [n, k]
  float* weights;        // [n, k]
  int32_t* order;        // [n*kk]
  int32_t* counts;       // [n_ids]
  int32_t* offsets;      // [n_ids + 1]
  int32_t* inv;          // [n*kk]
  int32_t* active;       // [n_ids]
  int32_t* n_active;
  int32_t* zero;         // counters to clear
  int n_zero;
};

template <int EPL>
__global__ __launch_bounds__(1024) void route_dispatch_kernel(const RouteDecodeArgs a) {
  __shared__ int s_ids[kMaxRows];
  __shared__ int s_cnt[kMaxIds];
  __shared__ int s_off[kMaxIds];
  __shared__ int s_tmp[16];
  __shared__ float s_tv[16][kMaxK], s_tx[16][kMaxK], s_ov[16][kMaxK], s_ox[16][kMaxK];
  __shared__ int s_ti[16][kMaxK], s_oi[16][kMaxK];
  __shared__ float s_c[16][512];  // sigmoid group scan (E <= 512)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int e = a.e, k = a.k, kk = a.kk;
  const int epl = (e + 63) / 64;
  const int n_ids = e + (kk > k ? 1 : 0);

  for (int i = tid; i < a.n_zero; i += 1024) a.zero[i] = 0;
  for (int i = tid; i < n_ids; i += 1024) s_cnt[i] = 0;

  for (int t = wv; t < a.n; t += 16) {
    const float* row = a.logits + size_t(t) * e;
    float v[EPL], x[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int ei = lane + 64 * i;
      v[i] = (i < epl && ei < e) ? row[ei] : 0.0f;
      x[i] = 0.0f;
    }
    if (a.scoring == PMOE_SCORE_SOFTMAX) {
      wave_topk_radix<false, EPL>(v, epl, e, k, s_ov[wv], s_oi[wv], x, nullptr, s_tv[wv], s_ti[wv],
                             s_tx[wv]);
      const float m = s_ov[wv][0];
      float s = 0.0f;
      if (a.norm) {
        for (int j = 0; j < k; ++j) s = s + pexp(s_ov[wv][j] - m);
      } else {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (i < epl && lane + 64 * i < e) acc = acc + pexp(v[i] - m);
        s = wave_sum_bfly(acc);
      }
      if (lane < k) {
        a.inds[size_t(t) * k + lane] = s_oi[wv][lane];
        a.weights[size_t(t) * k + lane] = pexp(s_ov[wv][lane] - m) / s;
        s_ids[t * kk + lane] = s_oi[wv][lane];
      }
    } else {
      // sigmoid + correction bias, grouped selection
      float c[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int ei = lane + 64 * i;
        if (i < epl && ei < e) {
          x[i] = psigmoid(v[i]);
          c[i] = x[i] + a.bias[ei];
          s_c[wv][ei] = c[i];
        } else {
          c[i] = 0.0f;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (a.n_group > 1) {
        const int gs = e / a.n_group;
        float gscore[EPL];
        gscore[0] = 0.0f;
        if (lane < a.n_group) {
          float t1 = -__builtin_inff(), t2 = -__builtin_inff();
          for (int j = 0; j < gs; ++j) {
            const float xv = s_c[wv][lane * gs + j];
            if (xv > t1) {
              t2 = t1;
              t1 = xv;
            } else if (xv > t2) {
              t2 = xv;
            }
          }
          gscore[0] = t1 + t2;
        }
#pragma unroll
        for (int i = 1; i < EPL; ++i) gscore[i] = 0.0f;
        wave_topk_radix<false, EPL>(gscore, 1, a.n_group, a.topk_group, s_tv[wv] + 8, s_ti[wv] + 8,
                               x, nullptr, s_tv[wv], s_ti[wv], s_tx[wv]);
        uint64_t keep = 0;
        for (int j = 0; j < a.topk_group; ++j) keep |= 1ull << s_ti[wv][8 + j];
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          const int ei = lane + 64 * i;
          if (i < epl && ei < e && !((keep >> (ei / gs)) & 1ull)) c[i] = 0.0f;
        }
      }
      wave_topk_radix<true, EPL>(c, epl, e, k, s_ov[wv], s_oi[wv], x, s_ox[wv], s_tv[wv], s_ti[wv],
                            s_tx[wv]);
      float s = 0.0f;
      for (int j = 0; j < k; ++j) s = s + s_ox[wv][j];
      if (lane < k) {
        float w = s_ox[wv][lane];
        if (a.norm) w = w / s;
        w = w * a.scale;
        a.inds[size_t(t) * k + lane] = s_oi[wv][lane];
        a.weights[size_t(t) * k + lane] = w;
        s_ids[t * kk + lane] = s_oi[wv][lane];
      }
    }
    if (kk > k && lane == 0) s_ids[t * kk + k] = e;  // shared expert column
  }
  __syncthreads();

  // stable dispatch of the rows (ids are valid by construction)
  const int rows = a.n * kk;
  int my_e = -1, rank = 0;
  if (tid < rows) {
    my_e = s_ids[tid];
    atomicAdd(&s_cnt[my_e], 1);
    for (int j = 0; j < tid; ++j) rank += (s_ids[j] == my_e);
  }
  __syncthreads();
  {
    const int c = tid < n_ids ? s_cnt[tid] : 0;
    // exclusive scans over ids: offsets and the active list
    int incl = c, act_incl = c > 0 ? 1 : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, kWave);
      const int oa = __shfl_up(act_incl, off, kWave);
      if (lane >= off) {
        incl += o;
        act_incl += oa;
      }
    }
    __shared__ int s_wt[16], s_wa[16];
    if (lane == 63) {
      s_wt[wv] = incl;
      s_wa[wv] = act_incl;
    }
    __syncthreads();
    if (wv == 0) {
      int x1 = lane < 16 ? s_wt[lane] : 0, x2 = lane < 16 ? s_wa[lane] : 0;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const int o1 = __shfl_up(x1, off, kWave), o2 = __shfl_up(x2, off, kWave);
        if (lane >= off) {
          x1 += o1;
          x2 += o2;
        }
      }
      if (lane < 16) {
        s_wt[lane] = x1;
        s_wa[lane] = x2;
      }
    }
    __syncthreads();
    const int off_e = (wv > 0 ? s_wt[wv - 1] : 0) + incl - c;
    const int act_e = (wv > 0 ? s_wa[wv - 1] : 0) + act_incl - (c > 0 ? 1 : 0);
    if (tid < n_ids) {
      s_off[tid] = off_e;
      a.counts[tid] = c;
      a.offsets[tid] = off_e;
      if (c > 0) a.active[act_e] = tid;
    }
    if (tid == 0) {
      a.offsets[n_ids] = s_wt[15];
      *a.n_active = s_wa[15];
    }
    (void)s_tmp;
  }
  __syncthreads();
  if (tid < rows) {
    const int pos = s_off[my_e] + rank;
    a.order[pos] = tid;
    a.inv[tid] = pos;
  }
}

}  // namespace

// Route + dispatch for n <= 64 tokens.  shared: append the shared pseudo-id
// e as column k of every token.  zero/n_zero: int32 counters to clear.
int route_dispatch_decode(const float* logits, const float* bias, int scoring, int n, int e, int k,
                          int shared, int norm, int n_group, int topk_group, float scale,
                          int32_t* inds, float* weights, int32_t* order, int32_t* counts,
                          int32_t* offsets, int32_t* inv, int32_t* active, int32_t* n_active,
                          int32_t* zero, int n_zero, hipStream_t st) {
  const int kk = k + (shared ? 1 : 0);
  PMOE_REQUIRE(n > 0 && n <= kMaxTokens, "route_dispatch_decode: 1..64 tokens");
  PMOE_REQUIRE(e > 0 && e + 1 <= kMaxIds && k > 0 && k <= kMaxK && k <= e,
               "route_dispatch_decode: bad experts/top-k");
  PMOE_REQUIRE(n * kk <= kMaxRows, "route_dispatch_decode: too many rows");
  if (scoring == PMOE_SCORE_SIGMOID) {
    PMOE_REQUIRE(bias != nullptr, "route_dispatch_decode: sigmoid needs bias");
    PMOE_REQUIRE(e <= 512, "route_dispatch_decode: sigmoid scoring supports E <= 512");
    PMOE_REQUIRE(n_group >= 1 && n_group <= 64 && e % n_group == 0 && topk_group >= 1 &&
                     topk_group <= n_group && topk_group <= 8 &&
                     (n_group == 1 || e / n_group >= 2) && k <= (e / n_group) * topk_group,
                 "route_dispatch_decode: bad group configuration");
  }
  RouteDecodeArgs a{logits, bias, n, e, k, kk, norm, n_group, topk_group, scale, scoring,
                    inds, weights, order, counts, offsets, inv, active, n_active, zero, n_zero};
  ProfScope prof_scope(K_ROUTE_SELECT, st);
  const int epl = (e + 63) / 64;
  if (epl <= 2)
    route_dispatch_kernel<2><<<1, 1024, 0, st>>>(a);
  else if (epl <= 4)
    route_dispatch_kernel<4><<<1, 1024, 0, st>>>(a);
  else if (epl <= 8)
    route_dispatch_kernel<8><<<1, 1024, 0, st>>>(a);
  else
    route_dispatch_kernel<16><<<1, 1024, 0, st>>>(a);
  PMOE_LAUNCH_CHECK("route_dispatch_kernel");
  return PMOE_OK;
}

}  // namespace pmoe
