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

template <int BITS, int LPR, int GPL, int MT, bool DUAL>
__global__ __launch_bounds__(256) void qgemv_kernel(const GemvArgs a) {
  constexpr int RPW = 64 / LPR;  // rows per wave step
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

  const int row0 = blockIdx.x * a.rows_per_block;
  const int rows_per_wave = a.rows_per_block / 4;
  const int wrow0 = row0 + wave * rows_per_wave;
  const int steps = rows_per_wave / RPW;

  if (slot < 0) {
    // Not resident: this expert contributes exact zero rows.
    for (int m = 0; m < m_total; ++m) {
      const int r = rlist[m];
      for (int i = threadIdx.x; i < a.rows_per_block; i += 256) {
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

  for (int m0 = 0; m0 < m_total; m0 += MT) {
    GroupAct<BITS> act[MT][GPL];
    int rr[MT];
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
    for (int st = 0; st < steps; ++st) {
      const int o = wrow0 + st * RPW + rsub;
      const bool row_ok = o < a.rows_out;
      const int oc = row_ok ? o : a.rows_out - 1;
      float p0[MT], p1[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) p0[t] = p1[t] = 0.0f;
#pragma unroll
      for (int j = 0; j < GPL; ++j) {
        const int g = sub + LPR * j;
        if (g < groups) {
          GroupW<BITS> q0, q1;
          load_group_w<BITS>(W0 + size_t(oc) * wpr, S0 + size_t(oc) * groups,
                             B0 + size_t(oc) * groups, g, q0);
          if (DUAL)
            load_group_w<BITS>(W1 + size_t(oc) * wpr, S1 + size_t(oc) * groups,
                               B1 + size_t(oc) * groups, g, q1);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            p0[t] = group_term(group_dot<BITS>(q0, act[t][j]), q0.s, q0.b, act[t][j].sum, p0[t]);
            if (DUAL)
              p1[t] =
                  group_term(group_dot<BITS>(q1, act[t][j]), q1.s, q1.b, act[t][j].sum, p1[t]);
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
        if (sub == t && row_ok && m0 + t < m_total) {
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

struct Shape {
  int lpr, gpl;
};

// Lanes per row (a power of two) and groups per lane for a row of `groups`
// quant groups: a lane owns groups sub, sub+LPR, ... so x for its groups stays
// in registers across every row the wave visits.
Shape pick_shape(int groups) {
  if (groups == 8 || groups == 16 || groups == 32 || groups == 64) return {groups, 1};
  if (groups % 8 == 0 && groups / 8 <= 4) return {8, groups / 8};
  if (groups <= 64) return {64, 1};
  if (groups <= 128) return {64, 2};
  return {0, 0};
}

template <int BITS, int LPR, int GPL, bool DUAL>
int launch_mt(const GemvArgs& a, int max_rows_per_expert, dim3 grid, hipStream_t st) {
  // activation registers: MT tokens x GPL groups x 33 VGPRs, capped at 4 groups
  constexpr int kCap = 4 / GPL;
  if (max_rows_per_expert <= 1 || kCap == 1) {
    qgemv_kernel<BITS, LPR, GPL, 1, DUAL><<<grid, 256, 0, st>>>(a);
  } else if (max_rows_per_expert <= 2 || kCap == 2) {
    qgemv_kernel<BITS, LPR, GPL, (kCap >= 2 ? 2 : 1), DUAL><<<grid, 256, 0, st>>>(a);
  } else {
    qgemv_kernel<BITS, LPR, GPL, (kCap >= 4 ? 4 : 1), DUAL><<<grid, 256, 0, st>>>(a);
  }
  PMOE_LAUNCH_CHECK("qgemv_kernel");
  return PMOE_OK;
}

template <int BITS, bool DUAL>
int launch_shape(const GemvArgs& a, Shape sh, int max_rows_per_expert, dim3 grid,
                 hipStream_t st) {
#define PMOE_SHAPE(L, G) \
  if (sh.lpr == L && sh.gpl == G) return launch_mt<BITS, L, G, DUAL>(a, max_rows_per_expert, grid, st);
  PMOE_SHAPE(64, 1)
  PMOE_SHAPE(64, 2)
  PMOE_SHAPE(8, 1)
  PMOE_SHAPE(8, 2)
  PMOE_SHAPE(8, 3)
  PMOE_SHAPE(8, 4)
  PMOE_SHAPE(16, 1)
  PMOE_SHAPE(32, 1)
#undef PMOE_SHAPE
  return fail(PMOE_EINVAL, "qgemv: unsupported row shape");
}

}  // namespace

// One grouped projection launch.  max_experts bounds the number of active
// experts (grid.y); max_rows_per_expert bounds the rows any expert serves.
int qgemv(const GemvArgs& a, int bits, bool dual, int max_experts, int max_rows_per_expert,
          hipStream_t st) {
  const int groups = a.cols / 64;
  PMOE_REQUIRE(a.cols % 64 == 0 && groups > 0, "qgemv: input dim must be a multiple of 64");
  const Shape sh = pick_shape(groups);
  PMOE_REQUIRE(sh.lpr > 0, "qgemv: input dim too large (max 8192)");
  PMOE_REQUIRE(a.rows_per_block % (4 * (64 / sh.lpr)) == 0, "qgemv: bad rows_per_block");
  if (max_experts <= 0 || a.rows_out <= 0) return PMOE_OK;
  dim3 grid((a.rows_out + a.rows_per_block - 1) / a.rows_per_block, max_experts);
  ProfScope prof_scope(dual ? K_GATEUP : K_DOWN, st);
  if (bits == 4)
    return dual ? launch_shape<4, true>(a, sh, max_rows_per_expert, grid, st)
                : launch_shape<4, false>(a, sh, max_rows_per_expert, grid, st);
  if (bits == 6)
    return dual ? launch_shape<6, true>(a, sh, max_rows_per_expert, grid, st)
                : launch_shape<6, false>(a, sh, max_rows_per_expert, grid, st);
  return fail(PMOE_EINVAL, "qgemv: bits must be 4 or 6");
}

// Rows per block: a multiple of 4 waves x rows-per-wave-step, sized so the
// grid has about `target` blocks when every possible expert is active.
int qgemv_rows_per_block(int cols, int rows_out, int max_experts, int target) {
  const Shape sh = pick_shape(cols / 64);
  const int unit = 4 * (64 / (sh.lpr > 0 ? sh.lpr : 64));
  long want = (long(rows_out) * max_experts + target - 1) / target;
  long r = (want + unit - 1) / unit * unit;
  if (r < unit) r = unit;
  if (r > 16L * unit) r = 16L * unit;
  return int(r);
}

}  // namespace pmoe
