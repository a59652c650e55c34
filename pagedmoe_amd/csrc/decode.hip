// Grouped dequant-GEMV for decode-sized batches (few rows per expert).
//
// Replaces the three mx.gather_qmm calls of the slab path (_run_slab ->
// _slab_rows -> _gather_proj, streaming.py:587-641 and :504-536) and the
// SwiGLU between them (streaming.py:640).  One launch computes a projection
// for every active expert at once: blockIdx.y picks the expert (ascending id,
// from the dispatch), blockIdx.x a tile of output rows, and each wave walks its
// rows with every lane owning whole 64-value quant groups of the row.
//
// Per lane and group: the packed weight words arrive as 16-byte loads, each
// 32-bit word is turned into bf16 pairs (128+q) with one and/or (4-bit) or a
// funnel shift (6-bit), and v_dot2_f32_bf16 accumulates x*(128+q) in fp32.
// With xs = sum of the group's x, the group's contribution is
//   s*sum(x*q) + b*xs = s*acc + (b - 128*s)*xs,
// so dequantised weights are never materialised.  Rows are reduced across
// their LPR lanes with an xor butterfly.  The gate/up launch (DUAL) computes
// both projections of a row together and writes h = silu(g)*u as bf16.
#include "pmoe_internal.h"
#include "pmoe_kernels.h"

namespace pmoe {

namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), c, false);
}

// Activations of one 64-value group, pre-arranged as the bf16 pairs the
// weight words of that group are unpacked into, plus the group sum.
template <int BITS>
struct GroupAct {
  uint32_t p[32];
  float sum;
};

// Load 64 bf16 starting at src (16-byte aligned) into pair order.
template <int BITS>
__device__ __forceinline__ void load_group_act(const uint16_t* src, GroupAct<BITS>& a) {
  const uint4* v = reinterpret_cast<const uint4*>(src);
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint4 d = v[c];
    s += bf16lo(d.x) + bf16hi(d.x) + bf16lo(d.y) + bf16hi(d.y) + bf16lo(d.z) + bf16hi(d.z) +
         bf16lo(d.w) + bf16hi(d.w);
    if (BITS == 4) {
      // word c of the group holds values 8c..8c+7; pair i is (x_{8c+i}, x_{8c+i+4})
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

template <int BITS>
struct GroupW {
  static constexpr int kWords = 64 * BITS / 32;
  uint32_t w[kWords];
  float s, b;
};

template <int BITS>
__device__ __forceinline__ void load_group_w(const uint32_t* wrow, const uint16_t* srow,
                                             const uint16_t* brow, int g, GroupW<BITS>& q) {
  constexpr int kWords = GroupW<BITS>::kWords;
  const u32x4* v = reinterpret_cast<const u32x4*>(wrow + size_t(g) * kWords);
#pragma unroll
  for (int c = 0; c < kWords / 4; ++c) {
    const u32x4 d = __builtin_nontemporal_load(v + c);
    q.w[4 * c + 0] = d.x;
    q.w[4 * c + 1] = d.y;
    q.w[4 * c + 2] = d.z;
    q.w[4 * c + 3] = d.w;
  }
  q.s = bf16f(srow[g]);
  q.b = bf16f(brow[g]);
}

// sum over the group of x*(128+q)
template <int BITS>
__device__ __forceinline__ float group_dot(const GroupW<BITS>& q, const GroupAct<BITS>& a) {
  float acc = 0.0f;
  if (BITS == 4) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t w = q.w[c];
      acc = dot2(a.p[4 * c + 0], (w & 0x000F000Fu) | 0x43004300u, acc);
      acc = dot2(a.p[4 * c + 1], ((w >> 4) & 0x000F000Fu) | 0x43004300u, acc);
      acc = dot2(a.p[4 * c + 2], ((w >> 8) & 0x000F000Fu) | 0x43004300u, acc);
      acc = dot2(a.p[4 * c + 3], ((w >> 12) & 0x000F000Fu) | 0x43004300u, acc);
    }
  } else {
#pragma unroll
    for (int p = 0; p < 32; ++p) {
      const int bit = 12 * p;
      const int wi = bit >> 5, sh = bit & 31;
      uint32_t f;
      if (sh + 12 <= 32)
        f = q.w[wi] >> sh;
      else
        f = __builtin_amdgcn_alignbit(q.w[wi + 1], q.w[wi], sh);
      const uint32_t pr = (f & 0x3Fu) | ((f << 10) & 0x003F0000u) | 0x43004300u;
      acc = dot2(a.p[p], pr, acc);
    }
  }
  return acc;
}

__device__ __forceinline__ float group_term(float acc, float s, float b, float xs, float part) {
  return __builtin_fmaf(s, acc, __builtin_fmaf(b - 128.0f * s, xs, part));
}

// Rows per wave step RPW = 64/LPR; a wave owns R consecutive steps.  All of
// its packed weights (R steps x GPL groups x 1-2 projections) are requested
// before anything else, so every wave has its whole share of HBM traffic in
// flight while the activations are still arriving from L2.
template <int BITS, int LPR, int GPL, int MT, int R, bool DUAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 8))) void qgemv_kernel(
    const GemvArgs a) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % LPR;
  const int rsub = lane / LPR;
  const int u = blockIdx.y;
  if (u >= *a.n_active) return;
  const int e = a.active[u];
  const int slot = e < a.n_experts ? a.table[e] : a.shared_slot;
  const int m_total = a.counts[e];
  const int32_t* rlist = a.order + a.offsets[e];
  const int groups = a.cols / 64;
  const int wpr = a.cols * BITS / 32;
  const int row0 = blockIdx.x * (4 * R * RPW);
  const int wrow0 = row0 + wave * (R * RPW);

  if (slot < 0) {
    // Not resident: this expert contributes exact zero rows.
    for (int m = 0; m < m_total; ++m) {
      const int r = rlist[m];
      for (int i = threadIdx.x; i < 4 * R * RPW; i += 256) {
        const int o = row0 + i;
        if (o >= a.rows_out) break;
        if (a.out_f32)
          static_cast<float*>(a.out)[size_t(r) * a.out_stride + o] = 0.0f;
        else
          static_cast<uint16_t*>(a.out)[size_t(r) * a.out_stride + o] = 0;
      }
    }
    return;
  }
  const uint8_t* base = a.slab + size_t(slot) * a.expert_bytes;
  const uint32_t* W0 = reinterpret_cast<const uint32_t*>(base + a.p0.w);
  const uint16_t* S0 = reinterpret_cast<const uint16_t*>(base + a.p0.s);
  const uint16_t* B0 = reinterpret_cast<const uint16_t*>(base + a.p0.b);
  const uint32_t* W1 = reinterpret_cast<const uint32_t*>(base + a.p1.w);
  const uint16_t* S1 = reinterpret_cast<const uint16_t*>(base + a.p1.s);
  const uint16_t* B1 = reinterpret_cast<const uint16_t*>(base + a.p1.b);

  // Activations first (L2 hits), then the weight burst: vector loads retire
  // in order, so row 0 can start as soon as its own words have landed.
  GroupAct<BITS> act[MT][GPL];
  int rr[MT];
  auto load_act = [&](int m0) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = min(m0 + t, m_total - 1);
      rr[t] = rlist[m];
      const int arow = a.act_by_token ? rr[t] / a.kk : rr[t];
      const uint16_t* src = a.act + size_t(arow) * a.act_stride;
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const int g = min(sub + LPR * j, groups - 1);
        load_group_act<BITS>(src + size_t(g) * 64, act[t][j]);
      }
    }
  };
  load_act(0);
  __builtin_amdgcn_sched_barrier(0);
  GroupW<BITS> q0[R][GPL];
  GroupW<BITS> q1[DUAL ? R : 1][DUAL ? GPL : 1];
#pragma unroll
  for (int st = 0; st < R; ++st) {
    const int o = min(wrow0 + st * RPW + rsub, a.rows_out - 1);
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      const int g = min(sub + LPR * j, groups - 1);
      load_group_w<BITS>(W0 + size_t(o) * wpr, S0 + size_t(o) * groups, B0 + size_t(o) * groups,
                         g, q0[st][j]);
      if (DUAL)
        load_group_w<BITS>(W1 + size_t(o) * wpr, S1 + size_t(o) * groups,
                           B1 + size_t(o) * groups, g, q1[DUAL ? st : 0][DUAL ? j : 0]);
    }
  }

  __builtin_amdgcn_sched_barrier(0);

  for (int m0 = 0; m0 < m_total; m0 += MT) {
    if (m0 > 0) {
      load_act(m0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int st = 0; st < R; ++st) {
      // Opaque to the optimiser: without this the unpacked pairs of every
      // row are hoisted out of the token loop and spill.
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
#pragma unroll
        for (int c = 0; c < GroupW<BITS>::kWords; ++c) {
          asm volatile("" : "+v"(q0[st][j].w[c]));
          if (DUAL) asm volatile("" : "+v"(q1[DUAL ? st : 0][DUAL ? j : 0].w[c]));
        }
      }
      const int o = wrow0 + st * RPW + rsub;
      float p0[MT], p1[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) p0[t] = p1[t] = 0.0f;
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        if (sub + LPR * j < groups) {
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            p0[t] = group_term(group_dot<BITS>(q0[st][j], act[t][j]), q0[st][j].s, q0[st][j].b,
                               act[t][j].sum, p0[t]);
            if (DUAL) {
              const GroupW<BITS>& w1 = q1[DUAL ? st : 0][DUAL ? j : 0];
              p1[t] = group_term(group_dot<BITS>(w1, act[t][j]), w1.s, w1.b, act[t][j].sum, p1[t]);
            }
          }
        }
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const float g0 = group_sum<LPR>(p0[t]);
        float v = g0;
        if (DUAL) {
          const float u1 = group_sum<LPR>(p1[t]);
          v = silu_fast(g0) * u1;
        }
        if (sub == t && o < a.rows_out && m0 + t < m_total) {
          const size_t idx = size_t(rr[t]) * a.out_stride + o;
          if (a.out_f32)
            static_cast<float*>(a.out)[idx] = v;
          else
            static_cast<uint16_t*>(a.out)[idx] = f2bf(v);
        }
      }
    }
  }
}

// Down projection + weighted combine for the decode block path.
//
// Tile-major: block b owns output rows [b*T, b*T + T) of the hidden dim for
// every active expert; wave w takes experts w, w+4, ...  Each (flat row r,
// output o) value lands in LDS, and once all experts are done the block
// forms out[n, o] = sum_c w[n, c] * y[n*kk + c, o] for c = 0..kk-1 in that
// fixed order (shared expert last), so the combine needs no y buffer, no
// separate launch and no cross-block synchronisation, and every block does
// the same amount of work.
template <int BITS, int LPR, int GPL, int R>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 8))) void
down_combine_kernel(const GemvArgs a, const CombineArgs c) {
  constexpr int RPW = 64 / LPR;
  constexpr int T = R * RPW;
  extern __shared__ float s_y[];  // [rows][T]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % LPR;
  const int rsub = lane / LPR;
  const int row0 = blockIdx.x * T;
  const int groups = a.cols / 64;
  const int wpr = a.cols * BITS / 32;
  const int n_act = *a.n_active;

  for (int u = wave; u < n_act; u += 4) {
    const int e = a.active[u];
    const int slot = e < a.n_experts ? a.table[e] : a.shared_slot;
    const int m_total = a.counts[e];
    const int32_t* rlist = a.order + a.offsets[e];
    if (slot < 0) {
      for (int m = 0; m < m_total; ++m)
        for (int t = lane; t < T; t += 64) s_y[rlist[m] * T + t] = 0.0f;
      continue;
    }
    const uint8_t* base = a.slab + size_t(slot) * a.expert_bytes;
    const uint32_t* W0 = reinterpret_cast<const uint32_t*>(base + a.p0.w);
    const uint16_t* S0 = reinterpret_cast<const uint16_t*>(base + a.p0.s);
    const uint16_t* B0 = reinterpret_cast<const uint16_t*>(base + a.p0.b);
    GroupAct<BITS> act[GPL];
    int r = rlist[0];
#pragma unroll
    for (int j = 0; j < GPL; ++j) {
      const int g = min(sub + LPR * j, groups - 1);
      load_group_act<BITS>(a.act + size_t(r) * a.act_stride + size_t(g) * 64, act[j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    GroupW<BITS> q0[R][GPL];
#pragma unroll
    for (int st = 0; st < R; ++st) {
      const int o = min(row0 + st * RPW + rsub, a.rows_out - 1);
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const int g = min(sub + LPR * j, groups - 1);
        load_group_w<BITS>(W0 + size_t(o) * wpr, S0 + size_t(o) * groups,
                           B0 + size_t(o) * groups, g, q0[st][j]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    for (int m = 0; m < m_total; ++m) {
      if (m > 0) {
        r = rlist[m];
#pragma unroll
        for (int j = 0; j < GPL; ++j) {
          const int g = min(sub + LPR * j, groups - 1);
          load_group_act<BITS>(a.act + size_t(r) * a.act_stride + size_t(g) * 64, act[j]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int st = 0; st < R; ++st) {
#pragma unroll
        for (int j = 0; j < GPL; ++j)
#pragma unroll
          for (int cw = 0; cw < GroupW<BITS>::kWords; ++cw) asm volatile("" : "+v"(q0[st][j].w[cw]));
        float p0 = 0.0f;
#pragma unroll
        for (int j = 0; j < GPL; ++j)
          if (sub + LPR * j < groups)
            p0 = group_term(group_dot<BITS>(q0[st][j], act[j]), q0[st][j].s, q0[st][j].b,
                            act[j].sum, p0);
        const float y = group_sum<LPR>(p0);
        if (sub == 0) s_y[r * T + st * RPW + rsub] = y;
      }
    }
  }
  __syncthreads();
  // fixed-order combine of this tile
  for (int i = threadIdx.x; i < c.n * T; i += 256) {
    const int n = i / T, t = i - n * T;
    const int o = row0 + t;
    if (o >= a.rows_out) continue;
    float acc = 0.0f;
    for (int col = 0; col < a.kk; ++col) {
      float wt;
      if (col < c.k)
        wt = c.w[size_t(n) * c.k + col];
      else
        wt = c.shared_logit ? psigmoid(c.shared_logit[n]) : 1.0f;
      acc = __builtin_fmaf(wt, s_y[(n * a.kk + col) * T + t], acc);
    }
    c.out[size_t(n) * a.rows_out + o] = f2bf(acc);
  }
}

struct Shape {
  int lpr, gpl;
};

// Lanes per row: the smallest power of two >= groups (max 64), so a lane
// owns one quant group (two for rows of 65..128 groups) and keeps that
// group's activations in registers for every row the wave visits.
Shape pick_shape(int groups) {
  if (groups <= 0 || groups > 128) return {0, 0};
  int lpr = 8;
  while (lpr < groups && lpr < 64) lpr <<= 1;
  return {lpr, (groups + lpr - 1) / lpr};
}

// Row steps per wave: as many as fit next to the activations in a
// 3-waves-per-SIMD register budget (~150 VGPRs: MT*GPL*33 for activations,
// ~30 for addresses and sums, the rest for packed weights), at most 4.
template <int BITS, int GPL, int MT, bool DUAL>
constexpr int rows_r() {
  constexpr int per_step = GPL * (64 * BITS / 32 + 2) * (DUAL ? 2 : 1);
  constexpr int budget = 150 - 30 - MT * GPL * 33;
  constexpr int r = budget / per_step;
  return r < 1 ? 1 : (r > 4 ? 4 : r);
}

template <int BITS, int LPR, int GPL, int MT, bool DUAL>
int launch_one(const GemvArgs& a, int max_experts, hipStream_t st) {
  constexpr int R = rows_r<BITS, GPL, MT, DUAL>();
  const int rows_per_block = 4 * R * (64 / LPR);
  dim3 grid((a.rows_out + rows_per_block - 1) / rows_per_block, max_experts);
  qgemv_kernel<BITS, LPR, GPL, MT, R, DUAL><<<grid, 256, 0, st>>>(a);
  PMOE_LAUNCH_CHECK("qgemv_kernel");
  return PMOE_OK;
}

// One token per pass: the packed weights stay in registers across passes,
// so an expert serving several rows re-reads only its activations.
template <int BITS, int LPR, int GPL, bool DUAL>
int launch_mt(const GemvArgs& a, int, int max_experts, hipStream_t st) {
  return launch_one<BITS, LPR, GPL, 1, DUAL>(a, max_experts, st);
}

template <int BITS, bool DUAL>
int launch_shape(const GemvArgs& a, Shape sh, int max_rows_per_expert, int max_experts,
                 hipStream_t st) {
#define PMOE_SHAPE(L, G) \
  if (sh.lpr == L && sh.gpl == G) \
    return launch_mt<BITS, L, G, DUAL>(a, max_rows_per_expert, max_experts, st);
  PMOE_SHAPE(64, 1)
  PMOE_SHAPE(64, 2)
  PMOE_SHAPE(8, 1)
  PMOE_SHAPE(16, 1)
  PMOE_SHAPE(32, 1)
#undef PMOE_SHAPE
  return fail(PMOE_EINVAL, "qgemv: unsupported row shape");
}

template <int BITS, int LPR, int GPL>
int launch_down_combine(const GemvArgs& a, const CombineArgs& c, hipStream_t st) {
  constexpr int R = rows_r<BITS, GPL, 1, false>();
  constexpr int T = R * (64 / LPR);
  const size_t lds = size_t(c.n) * a.kk * T * sizeof(float);
  if (lds > 64 * 1024) return fail(PMOE_EINVAL, "down_combine: too many rows for one tile");
  dim3 grid((a.rows_out + T - 1) / T);
  down_combine_kernel<BITS, LPR, GPL, R><<<grid, 256, lds, st>>>(a, c);
  PMOE_LAUNCH_CHECK("down_combine_kernel");
  return PMOE_OK;
}

template <int BITS>
int down_combine_bits(const GemvArgs& a, const CombineArgs& c, Shape sh, hipStream_t st) {
#define PMOE_SHAPE(L, G) \
  if (sh.lpr == L && sh.gpl == G) return launch_down_combine<BITS, L, G>(a, c, st);
  PMOE_SHAPE(64, 1)
  PMOE_SHAPE(64, 2)
  PMOE_SHAPE(8, 1)
  PMOE_SHAPE(16, 1)
  PMOE_SHAPE(32, 1)
#undef PMOE_SHAPE
  return fail(PMOE_EINVAL, "down_combine: unsupported row shape");
}

}  // namespace

// Down projection of every active expert plus the fixed-order combine into
// c.out [n, rows_out] (decode block path).
int down_combine(const GemvArgs& a, const CombineArgs& c, int bits, hipStream_t st) {
  const Shape sh = pick_shape(a.cols / 64);
  PMOE_REQUIRE(a.cols % 64 == 0 && sh.lpr > 0, "down_combine: bad input dim");
  ProfScope prof_scope(K_DOWN, st);
  if (bits == 4) return down_combine_bits<4>(a, c, sh, st);
  if (bits == 6) return down_combine_bits<6>(a, c, sh, st);
  return fail(PMOE_EINVAL, "down_combine: bits must be 4 or 6");
}

// One grouped projection launch.  max_experts bounds the number of active
// experts (grid.y); max_rows_per_expert bounds the rows any expert serves.
int qgemv(const GemvArgs& a, int bits, bool dual, int max_experts, int max_rows_per_expert,
          hipStream_t st) {
  const int groups = a.cols / 64;
  PMOE_REQUIRE(a.cols % 64 == 0 && groups > 0, "qgemv: input dim must be a multiple of 64");
  const Shape sh = pick_shape(groups);
  PMOE_REQUIRE(sh.lpr > 0, "qgemv: input dim too large (max 8192)");
  if (max_experts <= 0 || a.rows_out <= 0) return PMOE_OK;
  ProfScope prof_scope(dual ? K_GATEUP : K_DOWN, st);
  if (bits == 4)
    return dual ? launch_shape<4, true>(a, sh, max_rows_per_expert, max_experts, st)
                : launch_shape<4, false>(a, sh, max_rows_per_expert, max_experts, st);
  if (bits == 6)
    return dual ? launch_shape<6, true>(a, sh, max_rows_per_expert, max_experts, st)
                : launch_shape<6, false>(a, sh, max_rows_per_expert, max_experts, st);
  return fail(PMOE_EINVAL, "qgemv: bits must be 4 or 6");
}

}  // namespace pmoe
