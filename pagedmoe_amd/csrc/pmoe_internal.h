// Shared device helpers and host error plumbing for libpmoe (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/pmoe.h"

// ---------------------------------------------------------------- host side

namespace pmoe {

void set_error(const std::string& msg);
void clear_error();

// Slot-safety ledger (copy_engine.cpp): true while recording.
bool ledger_on();
void ledger_put(int64_t kind, const void* who, int64_t a = 0, int64_t b = 0, int64_t c = 0);

inline int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

inline int hip_fail(hipError_t e, const char* what) {
  return fail(PMOE_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace pmoe

#define PMOE_HIP(call)                                   \
  do {                                                   \
    hipError_t e_ = (call);                              \
    if (e_ != hipSuccess) return pmoe::hip_fail(e_, #call); \
  } while (0)

#define PMOE_LAUNCH_CHECK(name)                          \
  do {                                                   \
    hipError_t e_ = hipGetLastError();                   \
    if (e_ != hipSuccess) return pmoe::hip_fail(e_, name); \
  } while (0)

#define PMOE_REQUIRE(cond, msg)                          \
  do {                                                   \
    if (!(cond)) return pmoe::fail(PMOE_EINVAL, msg);    \
  } while (0)

// ---------------------------------------------------------------- device side

namespace pmoe {

constexpr int kWave = 64;

__device__ __forceinline__ float bf16lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16f(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }

// float -> bf16 bits, round to nearest even (NaN -> quiet NaN).
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// exp(x) with separately rounded ops only: Cody-Waite reduction
// x = n*ln2 + r (ln2 = C1 + C2, C1 with 9 significant bits so n*C1 is exact)
// and the degree-7 Taylor series of e^r in Horner form.  The library is
// compiled with -ffp-contract=off, so every * and + below rounds on its own
// and the result is bit-identical to the CPU oracle's.
__device__ __forceinline__ float pexp(float x) {
  const float n = __builtin_rintf(x * 1.44269504f);
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
  int ni = (int)fminf(fmaxf(n, -200.0f), 200.0f);
  float out = __builtin_ldexpf(p, ni);
  return x < -86.0f ? 0.0f : out;
}

__device__ __forceinline__ float psigmoid(float x) { return 1.0f / (1.0f + pexp(-x)); }

// Value of lane (lane ^ D) -- an exact xor exchange without a trip through
// the LDS crossbar where the wave's cross-lane paths allow it: DPP quad
// permutes for D = 1, 2; DPP row shifts (left for lanes whose bit D is
// clear, right for the others) for D = 4, 8; ds_swizzle (xor mode) for 16;
// ds_bpermute for 32.
template <int D>
__device__ __forceinline__ float xor_lane(float v) {
  const int b = __float_as_int(v);
  int r;
  if constexpr (D == 1) {
    r = __builtin_amdgcn_update_dpp(b, b, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (D == 2) {
    r = __builtin_amdgcn_update_dpp(b, b, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (D == 4 || D == 8) {
    const int up = __builtin_amdgcn_update_dpp(b, b, 0x100 + D, 0xF, 0xF, false);  // row_shl
    const int dn = __builtin_amdgcn_update_dpp(b, b, 0x110 + D, 0xF, 0xF, false);  // row_shr
    r = (threadIdx.x & D) ? dn : up;
  } else if constexpr (D == 16) {
    r = __builtin_amdgcn_ds_swizzle(b, 0x401F);  // and 0x1f, xor 0x10
  } else {
    static_assert(D == 32, "xor_lane: D must be a power of two <= 32");
    r = __builtin_amdgcn_ds_bpermute(int((threadIdx.x & 63) ^ 32) << 2, b);
  }
  return __int_as_float(r);
}

// xor butterfly over the 64 lanes; every lane ends with the same bits.
__device__ __forceinline__ float wave_sum_bfly(float v) {
  v = v + xor_lane<32>(v);
  v = v + xor_lane<16>(v);
  v = v + xor_lane<8>(v);
  v = v + xor_lane<4>(v);
  v = v + xor_lane<2>(v);
  v = v + xor_lane<1>(v);
  return v;
}

// xor butterfly within aligned groups of W lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W >= 64) v = v + xor_lane<32>(v);
  if constexpr (W >= 32) v = v + xor_lane<16>(v);
  if constexpr (W >= 16) v = v + xor_lane<8>(v);
  if constexpr (W >= 8) v = v + xor_lane<4>(v);
  if constexpr (W >= 4) v = v + xor_lane<2>(v);
  if constexpr (W >= 2) v = v + xor_lane<1>(v);
  return v;
}

// Fast SiLU for the expert epilogue (tolerance-checked, not bit-exact).
__device__ __forceinline__ float silu_fast(float g) { return g / (1.0f + __expf(-g)); }

}  // namespace pmoe
