// Measurement probes (no reference counterpart): kernels of known HBM
// traffic, used by bench.py in the same run as the kernels they qualify.
//
//  * read_probe_kernel streams `bytes` with the access pattern of the expert
//    weight stream (16-byte loads, consecutive lanes on consecutive 16-byte
//    chunks, so one wave instruction covers 1 KB; four loads in flight per
//    lane; non-temporal, the data is read once) and folds every word into
//    one xor per thread so no load is dead.  Its bandwidth is the read
//    ceiling the decode roofline is compared with, and its FETCH_SIZE
//    counter, against the bytes it reads, is the counter's scale.
//  * copy_probe_kernel copies `bytes` (16-byte loads and stores); its
//    WRITE_SIZE against the bytes it writes is that counter's scale.
#include "pmoe_internal.h"

namespace {

constexpr int kProbeThreads = 256;
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
constexpr int kProbeUnroll = 4;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const v4u* __restrict__ src,
                                                                    size_t n16,
                                                                    uint32_t* __restrict__ sink) {
  const size_t stride = size_t(gridDim.x) * kProbeThreads;
  size_t i = size_t(blockIdx.x) * kProbeThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    v4u v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const v4u v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  sink[size_t(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

__global__ __launch_bounds__(kProbeThreads) void copy_probe_kernel(const uint4* __restrict__ src,
                                                                    uint4* __restrict__ dst,
                                                                    size_t n16) {
  const size_t stride = size_t(gridDim.x) * kProbeThreads;
  for (size_t i = size_t(blockIdx.x) * kProbeThreads + threadIdx.x; i < n16; i += stride)
    dst[i] = src[i];
}

int probe_blocks() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return cus * 8;
}

}  // namespace

extern "C" size_t pmoe_probe_sink_bytes(void) {
  return size_t(probe_blocks()) * kProbeThreads * sizeof(uint32_t);
}

extern "C" int pmoe_probe_read(const void* src, size_t bytes, void* sink, size_t sink_bytes,
                               void* stream) {
  pmoe::clear_error();
  PMOE_REQUIRE(src && sink, "probe_read: null pointer");
  PMOE_REQUIRE(bytes % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0,
               "probe_read: bytes and src must be 16-byte multiples");
  const int blocks = probe_blocks();
  PMOE_REQUIRE(blocks > 0, "probe_read: no device");
  PMOE_REQUIRE(sink_bytes >= size_t(blocks) * kProbeThreads * sizeof(uint32_t),
               "probe_read: sink smaller than pmoe_probe_sink_bytes()");
  read_probe_kernel<<<blocks, kProbeThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const v4u*>(src), bytes / 16, static_cast<uint32_t*>(sink));
  PMOE_LAUNCH_CHECK("read_probe_kernel");
  return PMOE_OK;
}

extern "C" int pmoe_probe_copy(void* dst, const void* src, size_t bytes, void* stream) {
  pmoe::clear_error();
  PMOE_REQUIRE(src && dst, "probe_copy: null pointer");
  PMOE_REQUIRE(bytes % 16 == 0 &&
                   (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 == 0,
               "probe_copy: bytes, src and dst must be 16-byte multiples");
  const int blocks = probe_blocks();
  PMOE_REQUIRE(blocks > 0, "probe_copy: no device");
  copy_probe_kernel<<<blocks, kProbeThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), static_cast<uint4*>(dst), bytes / 16);
  PMOE_LAUNCH_CHECK("copy_probe_kernel");
  return PMOE_OK;
}
