// Block-level routing helpers shared by the decode kernels.
//
// Every block of a decode GEMV launch recomputes the layer's routing from the
// fp32 router logits (a few hundred floats) instead of waiting for a separate
// routing launch.  The computation is deterministic and uses only separately
// rounded float ops, so every block, and the CPU oracle, get identical bits:
//   * top-k per token: k rounds of a wave-wide maximum of order-preserving
//     keys, ties to the lower expert id, picks sorted by (value desc, id
//     asc) -- softmax(+renorm) or sigmoid+bias with grouped selection and
//     routed scaling (tests/test_stream.py:191-196; streaming.py:2424-2442);
//   * active experts: a bitmap of the used ids, listed in ascending order;
//   * rows of an expert: the flat (token, slot) rows holding its id, in
//     ascending order -- the stable dispatch of streaming.py:794.
#pragma once

#include "pmoe_internal.h"

#ifndef PMOE_ROUTE_MARK
#define PMOE_ROUTE_MARK(i)  // debug builds: a timestamp after each block barrier
#endif

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
  float c[kRouteMaxSigE];  // sigmoid scoring: biased scores, read across lanes
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

// Block barrier that orders LDS only: waits for this wave's LDS operations
// (lgkmcnt), not for its global stores, so a device-scope store issued just
// before does not hold the whole block until it is acknowledged.
__device__ __forceinline__ void block_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Inverse of order_key (a zero of either sign comes back as +0).
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Maximum of v over the wave (all 64 lanes active), wave-uniform: DPP
// maxima within each row of 16 lanes (quad swaps, half-row and row
// mirrors), then the four row maxima by readlane.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}

// Pick j of a top-k, held by lane j.
struct Pick {
  float v;  // value
  int i;    // id
  float x;  // payload carried along
};

// Compare-exchange: a ends up the larger (DESC) or the smaller key, the
// payloads following their keys.
template <bool PAYLOAD>
__device__ __forceinline__ void key_cas(uint64_t& a, uint64_t& b, float& pa, float& pb,
                                        bool desc) {
  const bool sw = desc ? (b > a) : (a > b);
  const uint64_t ka = a;
  a = sw ? b : a;
  b = sw ? ka : b;
  if (PAYLOAD) {
    const float qa = pa;
    pa = sw ? pb : pa;
    pb = sw ? qa : pb;
  }
}

// Bitonic sort of a lane's N keys (N a power of two), largest first;
// every index is static, so the keys stay in registers.
template <int N, bool PAYLOAD>
__device__ __forceinline__ void sort_keys_desc(uint64_t (&key)[N], float (&pay)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) key_cas<PAYLOAD>(key[i], key[j], pay[i], pay[j], (i & size) == 0);
      }
}

// Top-k of per-lane values v[i] (id lane + 64*i, valid when id < n_valid,
// k <= n_valid), in the order of the 64-bit keys order_key(v) << 32 | ~id:
// the larger value first and, among equal values, the lower id (invalid
// entries hold key 0, below every valid key).  Each lane sorts its keys
// once, largest first.  A round takes the wave maximum of the lanes' first
// values (32-bit); when one lane holds it, that lane's first key is the
// pick, else the lowest id among the lanes holding it (a second 32-bit
// maximum, of ~id); the lane that held the pick drops it (shifts its
// list).  Lane j (< k) returns pick j; picks come out sorted by (value
// desc, id asc), and extra[i] of each pick is carried along when PAYLOAD.
// Registers and scalar ops only.
template <int EPL, bool PAYLOAD = true>
__device__ __forceinline__ Pick wave_topk(const float (&v)[EPL], int n_valid, int k,
                                          const float (&extra)[EPL]) {
  const int lane = threadIdx.x & 63;
  uint64_t key[EPL];
  float pay[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int id = lane + 64 * i;
    key[i] = id < n_valid ? (uint64_t(order_key(v[i])) << 32) | uint32_t(~uint32_t(id)) : 0;
    pay[i] = PAYLOAD ? extra[i] : 0.0f;
  }
  sort_keys_desc<EPL, PAYLOAD>(key, pay);
  Pick pk{0.0f, 0, 0.0f};
  for (int j = 0; j < k; ++j) {
    const uint32_t hv = uint32_t(key[0] >> 32), hl = uint32_t(key[0]);
    const uint32_t top = wave_max_u32(hv);
    const uint64_t at = wave_ballot(hv == top);
    const uint32_t lo = __popcll(at) == 1
                            ? __builtin_amdgcn_readlane(hl, __builtin_ctzll(at))
                            : wave_max_u32(hv == top ? hl : 0u);
    const int sel = int(~lo);
    const int sl = sel & 63;
    const float pv = key_value(top);
    const float px =
        PAYLOAD ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pay[0]), sl)) : 0.0f;
    if (lane == sl) {
#pragma unroll
      for (int i = 0; i + 1 < EPL; ++i) {
        key[i] = key[i + 1];
        if (PAYLOAD) pay[i] = pay[i + 1];
      }
      key[EPL - 1] = 0;
    }
    if (lane == j) pk = Pick{pv, sel, px};
  }
  return pk;
}

// Value of `v` in lane j (j wave-uniform).
__device__ __forceinline__ float lane_value(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
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
  // the shared gate's logit, requested with the routed ones (loaded after
  // the top-k it would be a second round trip)
  const bool sg = r.kk > k && r.shared_gate;
  const float sg_logit = sg ? load_logit<COHERENT>(row + e) : 0.0f;
  float wk = 0.0f;
  int ik = 0;
  if (r.scoring == PMOE_SCORE_SOFTMAX) {
    const Pick pk = wave_topk<EPL, false>(v, e, k, x);
    const float m = lane_value(pk.v, 0);
    // lane j < k holds exp(v_j - m); the sum runs in pick order j = 0..k-1
    const float ej = lane < k ? pexp(pk.v - m) : 0.0f;
    float s = 0.0f;
    if (r.norm) {
      for (int j = 0; j < k; ++j) s = s + lane_value(ej, j);
    } else {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (lane + 64 * i < e) acc = acc + pexp(v[i] - m);
      s = wave_sum_bfly(acc);
    }
    if (lane < k) {
      ik = pk.i;
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
      float gscore[1] = {0.0f}, gnone[1] = {0.0f};  // group `lane` (n_group <= 64)
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
      const Pick gp = wave_topk<1, false>(gscore, r.n_group, r.topk_group, gnone);
      uint64_t keep = 0;
      for (int j = 0; j < r.topk_group; ++j) keep |= 1ull << __builtin_amdgcn_readlane(gp.i, j);
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int ei = lane + 64 * i;
        if (ei < e && !((keep >> (ei / gs)) & 1ull)) c[i] = 0.0f;
      }
    }
    const Pick pk = wave_topk<EPL>(c, e, k, x);
    float s = 0.0f;
    for (int j = 0; j < k; ++j) s = s + lane_value(pk.x, j);
    if (lane < k) {
      float w = pk.x;
      if (r.norm) w = w / s;
      wk = w * r.scale;
      ik = pk.i;
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
    L.w[t * r.kk + k] = sg ? psigmoid(sg_logit) : 1.0f;
  }
}

// One token with sigmoid scoring, by all NW waves of the block, bit for bit
// route_token's (and so the oracle's) picks and weights: wave w takes the
// experts [w*cs, w*cs + cs), cs = ceil(E / NW) <= 64, which are routing
// group w when there are groups (n_group == NW).  Each wave forms its
// sigmoids and biased scores; with groups, its group's score is the sum of
// its two largest biased scores (wave maxima, a repeated maximum counting
// twice) and wave 0 keeps the top groups exactly as route_token does; the
// other groups' scores become 0.  Scores are ordered by 64-bit keys
// (order_key(score) << 32 | ~id: larger score first, lower id among
// equals).  Each wave ranks its own keys (a lane's rank = the wave's keys
// above its own) and its top k -- the global top k is among them -- go to
// LDS; wave 0 ranks those NW*k candidates: pick j is the one with j greater
// keys.  The weights are route_token's: sigmoid / (sum over the
// picks in pick order) * scale.
__host__ __device__ __forceinline__ bool sigmoid_one_ok(const RouteDev& r, int nw) {
  const int cs = (r.e + nw - 1) / nw;
  return r.n == 1 && r.scoring == PMOE_SCORE_SIGMOID && cs <= 64 && r.k <= kRouteMaxK &&
         nw * r.k <= 128 && (r.n_group == 1 || (r.n_group == nw && r.e % nw == 0));
}

template <int NW, bool COHERENT>
__device__ void route_sigmoid_one(const RouteDev& r, RouteLds& L, int32_t* inds_out,
                                  float* w_out) {
  __shared__ float s_gscore[NW];
  __shared__ uint64_t s_keep;
  __shared__ uint64_t s_key[NW][64];
  __shared__ uint64_t s_ck[NW * kRouteMaxK];
  __shared__ float s_cx[NW * kRouteMaxK];
  __shared__ float s_px[kRouteMaxK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int e = r.e, k = r.k;
  const int cs = (e + NW - 1) / NW;
  const int base = wv * cs;
  const int nv = max(0, min(cs, e - base));  // experts of this wave
  const int ei = base + lane;
  const bool mine = lane < nv;
  float x = 0.0f, c = 0.0f;
  if (mine) {
    x = psigmoid(load_logit<COHERENT>(r.logits + ei));
    c = x + r.bias[ei];
  }
  if (r.n_group > 1) {
    const uint32_t kc = mine ? order_key(c) : 0u;
    const uint32_t k1 = wave_max_u32(kc);
    const uint64_t at = wave_ballot(mine && kc == k1);
    float t2;
    if (__popcll(at) >= 2) {
      t2 = key_value(k1);
    } else {
      const uint32_t k2 = wave_max_u32(lane == int(__builtin_ctzll(at)) ? 0u : kc);
      t2 = k2 == 0u ? -__builtin_inff() : key_value(k2);
    }
    if (lane == 0) s_gscore[wv] = key_value(k1) + t2;
    block_lds_sync();
    if (wv == 0) {
      float gscore[1] = {lane < r.n_group ? s_gscore[lane] : 0.0f}, gnone[1] = {0.0f};
      const Pick gp = wave_topk<1, false>(gscore, r.n_group, r.topk_group, gnone);
      uint64_t keep = 0;
      for (int j = 0; j < r.topk_group; ++j) keep |= 1ull << __builtin_amdgcn_readlane(gp.i, j);
      if (lane == 0) s_keep = keep;
    }
    block_lds_sync();
    if (mine && !((s_keep >> wv) & 1ull)) c = 0.0f;  // group wv is not kept
  }
  {
    // this wave's top k by rank counts over its keys (each lane compares
    // its key with every key of the wave); rank j goes to candidate slot j
    const uint64_t K = mine ? (uint64_t(order_key(c)) << 32) | uint32_t(~uint32_t(ei)) : 0ull;
    s_key[wv][lane] = K;
    if (lane < k) s_ck[wv * k + lane] = 0ull;  // slots past the wave's experts
    wave_lds_sync();
    int rk = 0;
    for (int m = 0; m < nv; ++m) rk += s_key[wv][m] > K ? 1 : 0;
    if (mine && rk < k) {
      s_ck[wv * k + rk] = K;
      s_cx[wv * k + rk] = x;
    }
  }
  block_lds_sync();
  if (wv == 0) {
    const int nc = NW * k;
    const uint64_t K0 = lane < nc ? s_ck[lane] : 0ull;
    const uint64_t K1 = lane + 64 < nc ? s_ck[lane + 64] : 0ull;
    int r0 = 0, r1 = 0;
    for (int m = 0; m < nc; ++m) {
      const uint64_t km = s_ck[m];
      r0 += km > K0 ? 1 : 0;
      r1 += km > K1 ? 1 : 0;
    }
    int ik = 0;
    if (lane < nc && r0 < k) {
      s_px[r0] = s_cx[lane];
      L.ids[r0] = int(~uint32_t(K0));
    }
    if (lane + 64 < nc && r1 < k) {
      s_px[r1] = s_cx[lane + 64];
      L.ids[r1] = int(~uint32_t(K1));
    }
    wave_lds_sync();
    const float px = lane < k ? s_px[lane] : 0.0f;
    if (lane < k) ik = L.ids[lane];
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) sum = sum + lane_value(px, j);
    if (lane < k) {
      float w = px;
      if (r.norm) w = w / sum;
      const float wk = w * r.scale;
      L.w[lane] = wk;
      if (inds_out) {
        inds_out[lane] = ik;
        w_out[lane] = wk;
      }
    }
    if (r.kk > k && lane == 0) {
      L.ids[k] = e;  // shared expert column
      L.w[k] = r.shared_gate ? psigmoid(load_logit<COHERENT>(r.logits + e)) : 1.0f;
    }
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
  if (sigmoid_one_ok(r, NW)) {
    route_sigmoid_one<NW, COHERENT>(r, L, inds_out, w_out);
  } else {
    for (int t = wv; t < r.n; t += NW)
      route_token<EPL, COHERENT>(r, t, L, W[wv], inds_out, w_out);
  }
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

// Top-k selection of ONE token over at most 128 routed experts (softmax +
// renorm scoring), logits in LDS, with a block of at least 512 threads.
// Expert i is picked at rank #{j : K_j > K_i}, K = order_key << 32 | ~id
// (ties to the lower id), counted in 4 quarters of 32 keys each; picks
// come out in rank order -- the order of wave_topk (value descending, lower
// id first).  Wave 0 lists the picks (L.ids), the active experts in
// ascending id order (L.active, shared expert last) and their count; the
// weights are left to route_rank1_weights, so the selection the weight
// stream waits for is all that comes first.  Results are bit-identical to
// route_block's.
struct Rank1Lds {
  uint64_t key[128];
  int32_t part[4][128];  // counts over each quarter of the keys
};

__host__ __device__ __forceinline__ bool rank1_route_ok(const RouteDev& r) {
  return r.scoring == PMOE_SCORE_SOFTMAX && r.norm && r.n == 1 && r.e <= 128 && r.k <= r.e &&
         r.k <= kRouteMaxK;
}

__device__ __forceinline__ void route_rank1_select(const RouteDev& r, const float* lg,
                                                   RouteLds& L, Rank1Lds& R) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int e = r.e, k = r.k;
  if (tid < 128)
    R.key[tid] = tid < e ? (uint64_t(order_key(lg[tid])) << 32) | uint32_t(~tid) : 0ull;
  __syncthreads();
  PMOE_ROUTE_MARK(28);
  if (tid < 512) {
    // expert i against quarter q of the keys; q is the same for the whole
    // wave, so every read is one address broadcast to all lanes (quarters
    // sit 256 bytes apart, on the same banks: spread over a wave's lanes
    // they would conflict on every read)
    const int q = (tid >> 6) & 3, i = (tid & 63) | ((tid >> 8) << 6);
    const uint64_t ki = R.key[i];
    const ulonglong2* kv = reinterpret_cast<const ulonglong2*>(R.key + 32 * q);
    ulonglong2 kj[16];  // all 16 reads in flight before the first compare
#pragma unroll
    for (int c = 0; c < 16; ++c) kj[c] = kv[c];
    __builtin_amdgcn_sched_barrier(0);
    int cnt = 0;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      cnt += kj[c].x > ki ? 1 : 0;
      cnt += kj[c].y > ki ? 1 : 0;
    }
    R.part[q][i] = cnt;
  }
  __syncthreads();
  PMOE_ROUTE_MARK(29);
  if (tid < 64) {
    auto rank_of = [&](int i) {
      return i < e ? R.part[0][i] + R.part[1][i] + R.part[2][i] + R.part[3][i] : 0x7fffffff;
    };
    const int r0 = rank_of(lane), r1 = rank_of(lane + 64);
    const bool sel0 = r0 < k, sel1 = r1 < k;
    if (sel0) L.ids[r0] = lane;
    if (sel1) L.ids[r1] = lane + 64;
    const uint64_t b0 = wave_ballot(sel0), b1 = wave_ballot(sel1);
    const int n0 = __popcll(b0);
    if (sel0) L.active[lanes_below(b0)] = lane;
    if (sel1) L.active[n0 + lanes_below(b1)] = lane + 64;
    if (lane == 0) {
      const int n_act = n0 + __popcll(b1);
      if (r.kk > k) {  // shared expert column: id e, listed last
        L.ids[k] = e;
        L.active[n_act] = e;
      }
      L.n_active = n_act + (r.kk > k ? 1 : 0);
    }
  }
  __syncthreads();
  PMOE_ROUTE_MARK(30);
}

// The combine weights of route_rank1_select's picks, by wave 0, exactly as
// route_token computes them: w_j = exp(v_j - v_0) / sum over picks in pick
// order (shared expert: 1, or sigmoid of its gate logit).
__device__ __forceinline__ void route_rank1_weights(const RouteDev& r, const float* lg,
                                                    RouteLds& L, int32_t* inds_out,
                                                    float* w_out) {
  const int lane = threadIdx.x & 63;
  if (threadIdx.x >= 64) return;
  const int k = r.k;
  const int ik = lane < k ? L.ids[lane] : 0;
  const float pv = lane < k ? lg[ik] : 0.0f;
  const float m = lane_value(pv, 0);
  const float ej = lane < k ? pexp(pv - m) : 0.0f;
  float s = 0.0f;
  for (int j = 0; j < k; ++j) s = s + lane_value(ej, j);
  if (lane < k) {
    const float wk = ej / s;
    L.w[lane] = wk;
    if (inds_out) {
      inds_out[lane] = ik;
      w_out[lane] = wk;
    }
  }
  if (r.kk > k && lane == 0) L.w[k] = r.shared_gate ? psigmoid(lg[r.e]) : 1.0f;
}

// Routing record in global memory: what block (0, 0) of the gate/up launch
// (or the routing launch) publishes for the later launches: the LDS copy's
// rows, and its active list with the shared expert moved to the front.
// It also holds the slab slot of every active expert (slot[u] for
// active[u]), so a per-expert block of the later launches finds its weights
// without a dependent slot-table read.
struct RouteRecord {
  int32_t ids[kRouteMaxRows];
  float w[kRouteMaxRows];
  int32_t active[kRouteMaxIds];
  int32_t slot[kRouteMaxIds];
  int32_t n_active;
};

// table: expert id -> slot (-1: absent); id n_experts is the shared expert.
// The record lists the shared expert (last in L.active) first: its blocks
// carry a row of every token, the longest work of a per-expert launch, and
// the dispatcher starts blocks in blockIdx.y order, so they start first
// instead of running alone at the end.  The routed experts follow in
// ascending id order.
__device__ __forceinline__ void publish_route(const RouteLds& L, int rows, RouteRecord* g,
                                              const int32_t* table, int n_experts,
                                              int shared_slot) {
  for (int i = threadIdx.x; i < rows; i += blockDim.x) {
    g->ids[i] = L.ids[i];
    g->w[i] = L.w[i];
  }
  const int na = L.n_active;
  const int rot = na > 0 && L.active[na - 1] >= n_experts ? na - 1 : 0;
  for (int u = threadIdx.x; u < na; u += blockDim.x) {
    const int e = L.active[u + rot < na ? u + rot : u + rot - na];
    g->active[u] = e;
    g->slot[u] = e < n_experts ? table[e] : shared_slot;
  }
  if (threadIdx.x == 0) g->n_active = na;
}

// What a block working on the u-th active expert needs from the record: the
// active count and the expert's id and slot, uniform over the block, read
// through the scalar cache (invalidated at every dispatch, and the record was
// written by an earlier launch).  A scalar load does not queue behind the
// vector loads that the CU's other blocks have in flight, so the block knows
// its weights' address before its first vector load returns.  u may exceed
// the active count (the launch's grid covers the most experts a call can
// route); those entries are in bounds and unused.
struct RouteOne {
  int n_active, e, slot;
};

__device__ __forceinline__ RouteOne load_route_one(const RouteRecord* g, int u) {
  typedef const __attribute__((address_space(4))) int32_t ConstI32;
  RouteOne o;
  o.n_active = *(ConstI32*)(&g->n_active);
  o.e = *(ConstI32*)(g->active + u);
  o.slot = *(ConstI32*)(g->slot + u);
  return o;
}

// Flat rows (ascending) of the record whose id is `id`, gathered by one wave
// straight from the record into out[] (no LDS staging of the ids; a wave
// that gathers its own list needs no block barrier either).  Returns the
// count.
__device__ __forceinline__ int wave_rows_of_record(const RouteRecord* g, int rows, int id,
                                                   int32_t* out) {
  static_assert(kRouteMaxRows == 256, "four ids a lane");
  const int lane = threadIdx.x & 63;
  int v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 64 * i + lane;
    v[i] = r < rows ? g->ids[r] : -1;
  }
  int m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (64 * i >= rows) break;
    const bool hit = v[i] == id;
    const uint64_t mask = wave_ballot(hit);
    if (hit) out[m + lanes_below(mask)] = 64 * i + lane;
    m += __popcll(mask);
  }
  wave_lds_sync();
  return m;
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
