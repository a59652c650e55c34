// Affine group quantization format: quantize and dequantize kernels.
//
// Format (safetensors_index.py:8-25, bench/slab_probe.py:82): weight u32
// [rows, cols*bits/32] holding a little-endian bit stream per row (value i at
// stream bits [i*bits, i*bits+bits)), scales and biases bf16 [rows,
// cols/group], w = s*q + b.  A group of 64 values is 64*bits/32 whole words
// (8 for 4-bit, 12 for 6-bit), so one thread owns one group.
#include "pmoe_internal.h"

namespace pmoe {

namespace {

template <int BITS>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ w, int rows,
                                                       int cols, uint32_t* __restrict__ q,
                                                       uint16_t* __restrict__ scales,
                                                       uint16_t* __restrict__ biases) {
  constexpr int kGroup = 64;
  constexpr int kWords = kGroup * BITS / 32;
  const int groups = cols / kGroup;
  const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= size_t(rows) * groups) return;
  const size_t row = gid / groups;
  const int g = int(gid % groups);
  const float* src = w + row * cols + size_t(g) * kGroup;
  float lo = src[0], hi = src[0];
  for (int i = 1; i < kGroup; ++i) {
    lo = fminf(lo, src[i]);
    hi = fmaxf(hi, src[i]);
  }
  const float scale = (hi - lo) / float((1 << BITS) - 1);
  uint16_t sb = f2bf(scale);
  if (bf16f(sb) == 0.0f) sb = 0x3F80;  // zero scale -> 1.0
  const uint16_t bb = f2bf(lo);
  const float s = bf16f(sb), b = bf16f(bb);
  scales[row * groups + g] = sb;
  biases[row * groups + g] = bb;
  uint32_t words[kWords];
#pragma unroll
  for (int j = 0; j < kWords; ++j) words[j] = 0;
  for (int i = 0; i < kGroup; ++i) {
    float qf = __builtin_rintf((src[i] - b) / s);
    qf = fminf(fmaxf(qf, 0.0f), float((1 << BITS) - 1));
    const uint32_t qi = uint32_t(qf);
    const int pos = i * BITS;
    words[pos >> 5] |= qi << (pos & 31);
    if ((pos & 31) + BITS > 32) words[(pos >> 5) + 1] |= qi >> (32 - (pos & 31));
  }
  uint32_t* dst = q + row * (size_t(cols) * BITS / 32) + size_t(g) * kWords;
#pragma unroll
  for (int j = 0; j < kWords; ++j) dst[j] = words[j];
}

template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ q,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      int rows, int cols,
                                                      uint16_t* __restrict__ out) {
  constexpr int kGroup = 64;
  constexpr int kWords = kGroup * BITS / 32;
  const int groups = cols / kGroup;
  const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= size_t(rows) * groups) return;
  const size_t row = gid / groups;
  const int g = int(gid % groups);
  const uint32_t* src = q + row * (size_t(cols) * BITS / 32) + size_t(g) * kWords;
  uint32_t words[kWords + 1];
#pragma unroll
  for (int j = 0; j < kWords; ++j) words[j] = src[j];
  words[kWords] = 0;
  const float s = bf16f(scales[row * groups + g]);
  const float b = bf16f(biases[row * groups + g]);
  uint16_t* dst = out + row * cols + size_t(g) * kGroup;
#pragma unroll
  for (int i = 0; i < kGroup; ++i) {
    const int pos = i * BITS;
    const uint64_t pair = uint64_t(words[pos >> 5]) | (uint64_t(words[(pos >> 5) + 1]) << 32);
    const uint32_t qi = uint32_t(pair >> (pos & 31)) & ((1u << BITS) - 1);
    dst[i] = f2bf(__builtin_fmaf(s, float(qi), b));
  }
}

}  // namespace

int quantize(const float* w, int rows, int cols, int bits, int group, uint32_t* q,
             uint16_t* scales, uint16_t* biases, hipStream_t st) {
  PMOE_REQUIRE(w && q && scales && biases, "quantize: null pointer");
  PMOE_REQUIRE(group == 64, "quantize: only group size 64 is supported");
  PMOE_REQUIRE(bits == 4 || bits == 6, "quantize: bits must be 4 or 6");
  PMOE_REQUIRE(rows >= 0 && cols > 0 && cols % 64 == 0, "quantize: cols must be a multiple of 64");
  const size_t n = size_t(rows) * (cols / 64);
  if (n == 0) return PMOE_OK;
  const unsigned blocks = unsigned((n + 255) / 256);
  if (bits == 4)
    quantize_kernel<4><<<blocks, 256, 0, st>>>(w, rows, cols, q, scales, biases);
  else
    quantize_kernel<6><<<blocks, 256, 0, st>>>(w, rows, cols, q, scales, biases);
  PMOE_LAUNCH_CHECK("quantize_kernel");
  return PMOE_OK;
}

int dequant(const uint32_t* q, const uint16_t* scales, const uint16_t* biases, int rows,
            int cols, int bits, int group, uint16_t* out, hipStream_t st) {
  PMOE_REQUIRE(q && scales && biases && out, "dequant: null pointer");
  PMOE_REQUIRE(group == 64, "dequant: only group size 64 is supported");
  PMOE_REQUIRE(bits == 4 || bits == 6, "dequant: bits must be 4 or 6");
  PMOE_REQUIRE(rows >= 0 && cols > 0 && cols % 64 == 0, "dequant: cols must be a multiple of 64");
  const size_t n = size_t(rows) * (cols / 64);
  if (n == 0) return PMOE_OK;
  const unsigned blocks = unsigned((n + 255) / 256);
  if (bits == 4)
    dequant_kernel<4><<<blocks, 256, 0, st>>>(q, scales, biases, rows, cols, out);
  else
    dequant_kernel<6><<<blocks, 256, 0, st>>>(q, scales, biases, rows, cols, out);
  PMOE_LAUNCH_CHECK("dequant_kernel");
  return PMOE_OK;
}

}  // namespace pmoe

extern "C" int pmoe_quantize(const float* w, int rows, int cols, int bits, int group, uint32_t* q,
                             uint16_t* scales, uint16_t* biases, void* stream) {
  pmoe::clear_error();
  return pmoe::quantize(w, rows, cols, bits, group, q, scales, biases,
                        static_cast<hipStream_t>(stream));
}

extern "C" int pmoe_dequant(const uint32_t* q, const uint16_t* scales, const uint16_t* biases,
                            int rows, int cols, int bits, int group, uint16_t* out, void* stream) {
  pmoe::clear_error();
  return pmoe::dequant(q, scales, biases, rows, cols, bits, group, out,
                       static_cast<hipStream_t>(stream));
}
