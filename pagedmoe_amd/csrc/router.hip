// Router: logits GEMV/GEMM in a fixed fp32 summation order, then top-k.
//
// Replaces the mlx-lm router the reference taps (streaming.py:167-193) and the
// selection the block performs after it: softmax(precise) -> argpartition ->
// take -> renorm (restated tests/test_stream.py:191-196) or DeepSeek-V3's
// sigmoid + correction bias + grouped top-k + routed scaling (consumed
// streaming.py:2424-2442).
//
// Summation order of a logit (shared with the CPU oracle, bit for bit): see
// router_tile.h.
#include <type_traits>

#include "pmoe_internal.h"
#include "pmoe_kernels.h"
#include "route_common.h"
#include "router_tile.h"

namespace pmoe {

namespace {

constexpr int kMaxEPL = 16;    // experts per lane in the select kernels (E <= 1024)
constexpr int kMaxK = 16;

// One wave computes a TE x TN tile of logits (experts x tokens); see
// router_tile.h for the summation order and the load grouping.
template <int TE, int TN, int UNR, bool FULL>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ w_extra, const float* __restrict__ bias, int n, int d, int e,
    int n_w, float* __restrict__ out) {
  const int wave = threadIdx.x >> 6;
  const int e0 = (blockIdx.x * kRouterWaves + wave) * TE;
  const int n0 = blockIdx.y * TN;
  if (e0 >= e) return;
  router_tile<TE, TN, UNR, FULL, false>(x, w, w_extra, bias, n, d, e, n_w, out, e0, n0);
}

// (value, index) order used by every top-k here: larger value first, lower
// index first among equal values.  idx < 0 marks "nothing".
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  if (i < 0) return false;
  if (bi < 0) return true;
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
}

// K picks over the per-lane values v[i] (expert lane + 64*i); excluded bit i
// of `skip` means v[i] is not a candidate.  Picks are written to sel_v/sel_i.
__device__ __forceinline__ void wave_topk(const float (&v)[kMaxEPL], uint32_t skip, int epl,
                                          int k, float* sel_v, int* sel_i) {
  const int lane = threadIdx.x & 63;
  uint32_t taken = skip;
  for (int kk = 0; kk < k; ++kk) {
    float bv = 0.0f;
    int bi = -1;
#pragma unroll
    for (int i = 0; i < kMaxEPL; ++i) {
      if (i < epl && !((taken >> i) & 1u)) {
        const int ei = lane + 64 * i;
        if (better(v[i], ei, bv, bi)) {
          bv = v[i];
          bi = ei;
        }
      }
    }
    wave_argmax(bv, bi);
    if (bi >= 0 && (bi & 63) == lane) taken |= 1u << (bi >> 6);
    sel_v[kk] = bv;
    sel_i[kk] = bi;
  }
}

// Softmax top-k of one token per wave (rows of logits [n, e]): the picks of
// pmoe::wave_topk (each lane sorts its logits once; k rounds of a 32-bit
// wave maximum), which are those of the (value desc, id asc) order, then the
// weights exp(v - v_max) / s with s the sum over the picks in pick order
// (norm) or the wave butterfly over all logits.  The same arithmetic as the
// decode launches' routing (route_common.h route_token).
template <int EPL>
__global__ __launch_bounds__(256) void route_softmax_kernel(
    const float* __restrict__ logits, int n, int e, int k, int norm,
    int32_t* __restrict__ inds, float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  float v[EPL], none[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int ei = lane + 64 * i;
    v[i] = ei < e ? logits[size_t(row) * e + ei] : 0.0f;
    none[i] = 0.0f;
  }
  const Pick pk = pmoe::wave_topk<EPL, false>(v, e, k, none);
  const float m = lane_value(pk.v, 0);
  const float ej = lane < k ? pexp(pk.v - m) : 0.0f;
  float s = 0.0f;
  if (norm) {
    for (int j = 0; j < k; ++j) s = s + lane_value(ej, j);
  } else {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + 64 * i < e) acc = acc + pexp(v[i] - m);
    s = wave_sum_bfly(acc);
  }
  if (lane < k) {
    inds[size_t(row) * k + lane] = pk.i;
    weights[size_t(row) * k + lane] = ej / s;
  }
}

// One token: the block-parallel sigmoid routing of the decode launches
// (route_common.h route_sigmoid_one, 8 waves), the same picks and weights.
__global__ __launch_bounds__(512) void route_sigmoid_one_kernel(const RouteDev r, int32_t* inds,
                                                                float* weights) {
  __shared__ RouteLds L;
  route_sigmoid_one<8, false>(r, L, inds, weights);
}

__global__ __launch_bounds__(256) void route_sigmoid_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int n, int e,
    int n_group, int topk_group, int k, int norm, float scale, int32_t* __restrict__ inds,
    float* __restrict__ weights) {
  __shared__ float s_c[4][1024];
  __shared__ float s_sig[4][1024];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int row_raw = blockIdx.x * 4 + wv;
  const bool valid = row_raw < n;
  const int row = valid ? row_raw : n - 1;
  const int epl = (e + 63) / 64;
  float c[kMaxEPL];
  uint32_t skip = 0;
#pragma unroll
  for (int i = 0; i < kMaxEPL; ++i) {
    const int ei = lane + 64 * i;
    c[i] = 0.0f;
    if (i < epl && ei < e) {
      const float sg = psigmoid(logits[size_t(row) * e + ei]);
      c[i] = sg + bias[ei];
      s_c[wv][ei] = c[i];
      s_sig[wv][ei] = sg;
    } else if (i < epl) {
      skip |= 1u << i;
    }
  }
  __syncthreads();
  if (n_group > 1) {
    const int gs = e / n_group;
    float gv = 0.0f;
    int gi = -1;
    if (lane < n_group) {
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
      gv = t1 + t2;
      gi = lane;
    }
    // topk_group picks among the group scores (one per lane < n_group).
    uint64_t keep = 0;
    bool mine_taken = false;
    for (int kk = 0; kk < topk_group; ++kk) {
      float bv = gv;
      int bi = mine_taken ? -1 : gi;
      wave_argmax(bv, bi);
      if (bi >= 0) {
        keep |= 1ull << bi;
        if (bi == lane) mine_taken = true;
      }
    }
#pragma unroll
    for (int i = 0; i < kMaxEPL; ++i) {
      const int ei = lane + 64 * i;
      if (i < epl && ei < e && !((keep >> (ei / gs)) & 1ull)) c[i] = 0.0f;
    }
  }
  float sv[kMaxK];
  int si[kMaxK];
  wave_topk(c, skip, epl, k, sv, si);
  float wk[kMaxK];
  float s = 0.0f;
  for (int kk = 0; kk < k; ++kk) {
    wk[kk] = s_sig[wv][si[kk]];
    s = s + wk[kk];
  }
  if (!valid) return;
  for (int kk = lane; kk < k; kk += 64) {
    float wt = wk[kk];
    if (norm) wt = wt / s;
    wt = wt * scale;
    inds[size_t(row) * k + kk] = si[kk];
    weights[size_t(row) * k + kk] = wt;
  }
}

}  // namespace

int router_logits_ext(const uint16_t* x, const uint16_t* w, const uint16_t* w_extra,
                      const float* bias, int n, int d, int n_w, float* out, hipStream_t st) {
  PMOE_REQUIRE(x && w && out, "router_logits: null pointer");
  PMOE_REQUIRE(n >= 0 && d > 0 && n_w > 0, "router_logits: bad shape");
  PMOE_REQUIRE(d % 8 == 0, "router_logits: hidden must be a multiple of 8");
  if (n == 0) return PMOE_OK;
  const int e = n_w + (w_extra ? 1 : 0);
  ProfScope prof_scope(K_ROUTER_LOGITS, st);
  const bool full = d % 512 == 0;
  auto launch = [&](auto te, auto tn, auto unr, dim3 grid) {
    constexpr int TE = decltype(te)::value, TN = decltype(tn)::value, UNR = decltype(unr)::value;
    if (full)
      router_logits_kernel<TE, TN, UNR, true><<<grid, 256, 0, st>>>(x, w, w_extra, bias, n, d, e,
                                                                   n_w, out);
    else
      router_logits_kernel<TE, TN, UNR, false><<<grid, 256, 0, st>>>(x, w, w_extra, bias, n, d,
                                                                    e, n_w, out);
  };
  using I1 = std::integral_constant<int, 1>;
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  if (n >= 32 && e >= 16) {
    // one pass per group: the 4 x 8 tile's 12 loads a pass keep three waves
    // per SIMD; staging 4 passes (256 registers, one wave) took 64 -> 139 us
    // at 2048 tokens.  (A few columns -- a shared expert's gate -- take the
    // 1 x 4 tile below: a 4 x 8 tile would leave one wave of four busy.)
    dim3 grid((e + kRouterWaves * 4 - 1) / (kRouterWaves * 4), (n + 8 - 1) / 8);
    launch(I4{}, I8{}, I1{}, grid);
  } else if (n >= 4) {
    dim3 grid((e + kRouterWaves - 1) / kRouterWaves, (n + 4 - 1) / 4);
    launch(I1{}, I4{}, I8{}, grid);
  } else {
    dim3 grid((e + kRouterWaves - 1) / kRouterWaves, n);
    launch(I1{}, I1{}, I8{}, grid);
  }
  PMOE_LAUNCH_CHECK("router_logits_kernel");
  return PMOE_OK;
}

int router_logits(const uint16_t* x, const uint16_t* w, const float* bias, int n, int d, int e,
                  float* out, hipStream_t st) {
  return router_logits_ext(x, w, nullptr, bias, n, d, e, out, st);
}

int route_softmax(const float* logits, int n, int e, int k, int norm, int32_t* inds,
                  float* weights, hipStream_t st) {
  PMOE_REQUIRE(logits && inds && weights, "route_softmax_topk: null pointer");
  PMOE_REQUIRE(e > 0 && e <= 64 * kMaxEPL, "route_softmax_topk: experts must be 1..1024");
  PMOE_REQUIRE(k > 0 && k <= kMaxK && k <= e, "route_softmax_topk: k must be 1..min(16, E)");
  if (n <= 0) return PMOE_OK;
  ProfScope prof_scope(K_ROUTE_SELECT, st);
  const int epl = (e + 63) / 64;
  const dim3 grid((n + 3) / 4);
  if (epl <= 1)
    route_softmax_kernel<1><<<grid, 256, 0, st>>>(logits, n, e, k, norm, inds, weights);
  else if (epl <= 2)
    route_softmax_kernel<2><<<grid, 256, 0, st>>>(logits, n, e, k, norm, inds, weights);
  else if (epl <= 4)
    route_softmax_kernel<4><<<grid, 256, 0, st>>>(logits, n, e, k, norm, inds, weights);
  else if (epl <= 8)
    route_softmax_kernel<8><<<grid, 256, 0, st>>>(logits, n, e, k, norm, inds, weights);
  else
    route_softmax_kernel<16><<<grid, 256, 0, st>>>(logits, n, e, k, norm, inds, weights);
  PMOE_LAUNCH_CHECK("route_softmax_kernel");
  return PMOE_OK;
}

int route_sigmoid(const float* logits, const float* bias, int n, int e, int n_group,
                  int topk_group, int k, int norm, float scale, int32_t* inds, float* weights,
                  hipStream_t st) {
  PMOE_REQUIRE(logits && bias && inds && weights, "route_sigmoid_group_topk: null pointer");
  PMOE_REQUIRE(e > 0 && e <= 64 * kMaxEPL, "route_sigmoid_group_topk: experts must be 1..1024");
  PMOE_REQUIRE(k > 0 && k <= kMaxK && k <= e, "route_sigmoid_group_topk: k must be 1..min(16, E)");
  PMOE_REQUIRE(n_group >= 1 && n_group <= 64 && e % n_group == 0,
               "route_sigmoid_group_topk: n_group must divide E and be <= 64");
  PMOE_REQUIRE(topk_group >= 1 && topk_group <= n_group,
               "route_sigmoid_group_topk: topk_group must be 1..n_group");
  PMOE_REQUIRE(n_group == 1 || e / n_group >= 2,
               "route_sigmoid_group_topk: groups need at least 2 experts");
  PMOE_REQUIRE(k <= (e / n_group) * topk_group,
               "route_sigmoid_group_topk: k exceeds the experts of the kept groups");
  if (n <= 0) return PMOE_OK;
  ProfScope prof_scope(K_ROUTE_SELECT, st);
  RouteDev r{};
  r.logits = logits;
  r.ld = e;
  r.bias = bias;
  r.scoring = PMOE_SCORE_SIGMOID;
  r.n = n;
  r.e = e;
  r.k = k;
  r.kk = k;
  r.norm = norm;
  r.n_group = n_group;
  r.topk_group = topk_group;
  r.scale = scale;
  if (sigmoid_one_ok(r, 8)) {  // one token: every wave of a block on it
    route_sigmoid_one_kernel<<<1, 512, 0, st>>>(r, inds, weights);
    PMOE_LAUNCH_CHECK("route_sigmoid_one_kernel");
    return PMOE_OK;
  }
  route_sigmoid_kernel<<<(n + 3) / 4, 256, 0, st>>>(logits, bias, n, e, n_group, topk_group, k,
                                                    norm, scale, inds, weights);
  PMOE_LAUNCH_CHECK("route_sigmoid_kernel");
  return PMOE_OK;
}

}  // namespace pmoe

extern "C" int pmoe_router_logits(const void* x, const void* w, const float* logit_bias, int n,
                                  int d, int e, float* logits, void* stream) {
  pmoe::clear_error();
  return pmoe::router_logits(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                             logit_bias, n, d, e, logits, static_cast<hipStream_t>(stream));
}

extern "C" int pmoe_route_softmax_topk(const float* logits, int n, int e, int k,
                                       int norm_topk_prob, int32_t* inds, float* weights,
                                       void* stream) {
  pmoe::clear_error();
  return pmoe::route_softmax(logits, n, e, k, norm_topk_prob, inds, weights,
                             static_cast<hipStream_t>(stream));
}

extern "C" int pmoe_route_sigmoid_group_topk(const float* logits, const float* bias, int n,
                                             int e, int n_group, int topk_group, int k,
                                             int norm_topk_prob, float routed_scale,
                                             int32_t* inds, float* weights, void* stream) {
  pmoe::clear_error();
  return pmoe::route_sigmoid(logits, bias, n, e, n_group, topk_group, k, norm_topk_prob,
                             routed_scale, inds, weights, static_cast<hipStream_t>(stream));
}
