/* C restatement of the routed-expert hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (as a second implementation of the oracle's routing, which
 * must agree with oracle/pmoe_oracle.py bit for bit) and by bench.py's
 * cpu_baseline leg (the CPU time of one decode MoE layer on the host cores).
 * The product (pagedmoe_amd) never links or calls this.
 *
 * Semantics follow oracle/pmoe_oracle.py, which cites the reference file:line
 * of each step:
 *   router logits      streaming.py:167-193 (canonical fp32 lane order)
 *   softmax top-k      tests/test_stream.py:191-196, streaming.py:2443-2452
 *   sigmoid group top-k  streaming.py:2424-2442 (DeepSeek-V3 noaux_tc)
 *   expert FFN         streaming.py:504-536, :640 (gather_qmm + SwiGLU)
 *   combine            tests/test_stream.py:198
 * Compiled with -ffp-contract=off: every + and * rounds on its own unless an
 * fmaf is written.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define LANES 64
#define CHUNK 8

static inline float bf(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float pmo_pexp(float x) {
  const float n = rintf(x * 1.44269504f);
  float r = x - n * 0.693359375f;
  r = r - n * -2.12194440e-4f;
  float p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  float nc = fminf(fmaxf(n, -200.0f), 200.0f);
  float out = ldexpf(p, (int)nc);
  return x < -86.0f ? 0.0f : out;
}

static void butterfly(float* acc) {
  float tmp[LANES];
  for (int off = LANES / 2; off > 0; off >>= 1) {
    for (int l = 0; l < LANES; ++l) tmp[l] = acc[l] + acc[l ^ off];
    memcpy(acc, tmp, sizeof(tmp));
  }
}

/* logits[n*e + j] = canonical fp32 dot of x[n] and w[j] (+ bias[j]) */
void pmo_router_logits(const uint16_t* x, const uint16_t* w, const float* bias, int n, int d,
                       int e, float* out) {
  const int passes = (d + LANES * CHUNK - 1) / (LANES * CHUNK);
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < n; ++t)
    for (int j = 0; j < e; ++j) {
      float acc[LANES];
      for (int l = 0; l < LANES; ++l) {
        float a = 0.0f;
        for (int p = 0; p < passes; ++p)
          for (int c = 0; c < CHUNK; ++c) {
            const int col = p * LANES * CHUNK + l * CHUNK + c;
            if (col < d) a = fmaf(bf(x[(size_t)t * d + col]), bf(w[(size_t)j * d + col]), a);
          }
        acc[l] = a;
      }
      butterfly(acc);
      out[(size_t)t * e + j] = bias ? acc[0] + bias[j] : acc[0];
    }
}

/* indices of the k largest v[0..e) sorted descending, ties to the lower id */
static void topk_desc(const float* v, int e, int k, int32_t* idx) {
  for (int kk = 0; kk < k; ++kk) {
    int best = -1;
    for (int j = 0; j < e; ++j) {
      int taken = 0;
      for (int q = 0; q < kk; ++q) taken |= idx[q] == j;
      if (taken) continue;
      if (best < 0 || v[j] > v[best]) best = j;
    }
    idx[kk] = best;
  }
}

void pmo_softmax_topk(const float* logits, int n, int e, int k, int norm, int32_t* inds,
                      float* wts) {
  for (int t = 0; t < n; ++t) {
    const float* l = logits + (size_t)t * e;
    int32_t* id = inds + (size_t)t * k;
    topk_desc(l, e, k, id);
    const float m = l[id[0]];
    float s = 0.0f;
    if (norm) {
      for (int kk = 0; kk < k; ++kk) s = s + pmo_pexp(l[id[kk]] - m);
    } else {
      float acc[LANES] = {0};
      for (int j = 0; j < e; ++j) acc[j % LANES] = acc[j % LANES] + pmo_pexp(l[j] - m);
      butterfly(acc);
      s = acc[0];
    }
    for (int kk = 0; kk < k; ++kk) wts[(size_t)t * k + kk] = pmo_pexp(l[id[kk]] - m) / s;
  }
}

void pmo_sigmoid_group_topk(const float* logits, const float* bias, int n, int e, int n_group,
                            int topk_group, int k, int norm, float scale, int32_t* inds,
                            float* wts) {
  float* sig = (float*)malloc(sizeof(float) * e);
  float* c = (float*)malloc(sizeof(float) * e);
  float* gsc = (float*)malloc(sizeof(float) * (n_group > 0 ? n_group : 1));
  int32_t* gid = (int32_t*)malloc(sizeof(int32_t) * (n_group > 0 ? n_group : 1));
  for (int t = 0; t < n; ++t) {
    const float* l = logits + (size_t)t * e;
    for (int j = 0; j < e; ++j) {
      sig[j] = 1.0f / (1.0f + pmo_pexp(-l[j]));
      c[j] = sig[j] + bias[j];
    }
    if (n_group > 1) {
      const int gs = e / n_group;
      for (int g = 0; g < n_group; ++g) {
        float t1 = -INFINITY, t2 = -INFINITY;
        for (int j = 0; j < gs; ++j) {
          const float v = c[g * gs + j];
          if (v > t1) {
            t2 = t1;
            t1 = v;
          } else if (v > t2) {
            t2 = v;
          }
        }
        gsc[g] = t1 + t2;
      }
      topk_desc(gsc, n_group, topk_group, gid);
      for (int g = 0; g < n_group; ++g) {
        int keep = 0;
        for (int q = 0; q < topk_group; ++q) keep |= gid[q] == g;
        if (!keep)
          for (int j = 0; j < gs; ++j) c[g * gs + j] = 0.0f;
      }
    }
    int32_t* id = inds + (size_t)t * k;
    topk_desc(c, e, k, id);
    float s = 0.0f;
    for (int kk = 0; kk < k; ++kk) s = s + sig[id[kk]];
    for (int kk = 0; kk < k; ++kk) {
      float w = sig[id[kk]];
      if (norm) w = w / s;
      wts[(size_t)t * k + kk] = w * scale;
    }
  }
  free(sig);
  free(c);
  free(gsc);
  free(gid);
}

/* One quantized projection y[o] = sum_i x[i] * (s*q + b), rows [0, rows).
 * Row-parallel; x fp32 [cols]. */
static void qproj(const uint32_t* w, const uint16_t* s, const uint16_t* b, int rows, int cols,
                  int bits, const float* x, const float* xs, float* y) {
  const int groups = cols / 64;
  const int wpr = cols * bits / 32;
  const uint32_t mask = (1u << bits) - 1u;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < rows; ++o) {
    const uint32_t* wr = w + (size_t)o * wpr;
    float acc = 0.0f;
    for (int g = 0; g < groups; ++g) {
      const uint32_t* wg = wr + (size_t)g * (64 * bits / 32);
      const float* xg = x + (size_t)g * 64;
      float qd = 0.0f;
      if (bits == 4) {
        for (int j = 0; j < 8; ++j) {
          const uint32_t v = wg[j];
          for (int c = 0; c < 8; ++c) qd = fmaf(xg[8 * j + c], (float)((v >> (4 * c)) & 15u), qd);
        }
      } else {
        for (int i = 0; i < 64; ++i) {
          const int pos = i * bits;
          uint64_t pair = wg[pos >> 5];
          if ((pos >> 5) + 1 < 64 * bits / 32) pair |= (uint64_t)wg[(pos >> 5) + 1] << 32;
          qd = fmaf(xg[i], (float)((uint32_t)(pair >> (pos & 31)) & mask), qd);
        }
      }
      acc = fmaf(bf(s[(size_t)o * groups + g]), qd, fmaf(bf(b[(size_t)o * groups + g]), xs[g], acc));
    }
    y[o] = acc;
  }
}

typedef struct {
  const uint32_t* w[3];  /* gate, up, down */
  const uint16_t* s[3];
  const uint16_t* b[3];
} pmo_expert;

/* FFN of one token on one expert: y[d] = down(silu(gate x) * up x). */
void pmo_expert_ffn(const pmo_expert* ex, const float* x, int d, int inter, int bits,
                    float* y, float* scratch) {
  float* g = scratch;
  float* u = g + inter;
  float* h = u + inter;
  float* xs = h + inter;
  float* hs = xs + d / 64;
  for (int q = 0; q < d / 64; ++q) {
    float a = 0.0f;
    for (int i = 0; i < 64; ++i) a += x[q * 64 + i];
    xs[q] = a;
  }
  qproj(ex->w[0], ex->s[0], ex->b[0], inter, d, bits, x, xs, g);
  qproj(ex->w[1], ex->s[1], ex->b[1], inter, d, bits, x, xs, u);
  for (int i = 0; i < inter; ++i) h[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
  for (int q = 0; q < inter / 64; ++q) {
    float a = 0.0f;
    for (int i = 0; i < 64; ++i) a += h[q * 64 + i];
    hs[q] = a;
  }
  qproj(ex->w[2], ex->s[2], ex->b[2], d, inter, bits, h, hs, y);
}

/* Scratch floats needed by pmo_moe_decode. */
size_t pmo_scratch_floats(int d, int inter) {
  return (size_t)3 * inter + d / 64 + inter / 64 + (size_t)2 * d + 64;
}

/* One decode MoE layer for n tokens: canonical router, softmax top-k,
 * experts, fp32 combine.  experts[e] gives each expert's components.  out
 * fp32 [n, d]; inds/wts [n, k]. */
void pmo_moe_decode(const uint16_t* x_bits, const uint16_t* gate_w, int n, int d, int n_exp,
                    int inter, int k, int bits, const pmo_expert* experts, float* logits,
                    int32_t* inds, float* wts, float* out, float* scratch) {
  pmo_router_logits(x_bits, gate_w, NULL, n, d, n_exp, logits);
  pmo_softmax_topk(logits, n, n_exp, k, 1, inds, wts);
  float* xf = scratch + 3 * (size_t)inter + d / 64 + inter / 64;
  float* y = xf + d;
  for (int t = 0; t < n; ++t) {
    for (int i = 0; i < d; ++i) xf[i] = bf(x_bits[(size_t)t * d + i]);
    float* o = out + (size_t)t * d;
    for (int i = 0; i < d; ++i) o[i] = 0.0f;
    for (int kk = 0; kk < k; ++kk) {
      const int e = inds[(size_t)t * k + kk];
      pmo_expert_ffn(&experts[e], xf, d, inter, bits, y, scratch);
      const float w = wts[(size_t)t * k + kk];
      for (int i = 0; i < d; ++i) o[i] = fmaf(w, y[i], o[i]);
    }
  }
}

int pmo_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
