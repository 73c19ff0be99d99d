// Streaming probes (diagnostic, no counterpart in the reference): the rates
// at which this part reads and copies large contiguous buffers with 16-byte
// lane accesses -- the ceilings that the bandwidth-bound kernels' figures
// (writer, W4A16 MoE weights, indexer keys) are read against.
//
// Grid-stride loops, kUnroll 16-byte loads per lane in flight per pass, one
// launch configuration per form: the fastest of grids 2048..16384 x unroll
// 4/8 measured on one MI355X over 2 GiB (plain read 8192 x 8: 6.3 TB/s;
// non-temporal read 16384 x 8: 7.1 TB/s; non-temporal copy 16384 x 4: 5.8
// TB/s of read + write bytes).
#include "glm53_common.h"

namespace glm53 {
namespace {

constexpr int kProbeThreads = 256;

template <int kUnroll, bool kNt>
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                                    u32x4* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads * kUnroll;
  uint32_t acc = 0;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kProbeThreads * kUnroll + threadIdx.x; base < n16;
       base += stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int64_t i = base + static_cast<int64_t>(u) * kProbeThreads;
      v[u] = i < n16 ? (kNt ? __builtin_nontemporal_load(src + i) : src[i]) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  // a data-dependent store the compiler cannot drop: keeps every load
  if (acc == 0x9E3779B9u) sink[0] = u32x4{acc, acc, acc, acc};
}

template <int kUnroll>
__global__ __launch_bounds__(kProbeThreads) void stream_copy_kernel(const u32x4* __restrict__ src,
                                                                    u32x4* __restrict__ dst, int64_t n16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads * kUnroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kProbeThreads * kUnroll + threadIdx.x; base < n16;
       base += stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int64_t i = base + static_cast<int64_t>(u) * kProbeThreads;
      if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int64_t i = base + static_cast<int64_t>(u) * kProbeThreads;
      if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
}

}  // namespace
}  // namespace glm53

using namespace glm53;

extern "C" int glm53_stream_probe(int kind, const void* src, void* dst, int64_t bytes, void* stream) {
  if (kind != GLM53_PROBE_READ && kind != GLM53_PROBE_READ_NT && kind != GLM53_PROBE_COPY_NT)
    return GLM53_ERR_BAD_SHAPE;
  if (!src || !dst) return GLM53_ERR_NULL_POINTER;
  if (bytes < 16 || bytes % 16) return GLM53_ERR_BAD_SHAPE;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) return GLM53_ERR_MISALIGNED;
  const auto st = static_cast<hipStream_t>(stream);
  const auto s = static_cast<const u32x4*>(src);
  const auto d = static_cast<u32x4*>(dst);
  const int64_t n16 = bytes / 16;
  (void)hipGetLastError();
  switch (kind) {
    case GLM53_PROBE_READ:
      hipLaunchKernelGGL((stream_read_kernel<8, false>), dim3(8192), dim3(kProbeThreads), 0, st, s, n16, d);
      break;
    case GLM53_PROBE_READ_NT:
      hipLaunchKernelGGL((stream_read_kernel<8, true>), dim3(16384), dim3(kProbeThreads), 0, st, s, n16, d);
      break;
    default:   // GLM53_PROBE_COPY_NT
      hipLaunchKernelGGL((stream_copy_kernel<4>), dim3(16384), dim3(kProbeThreads), 0, st, s, d, n16);
      break;
  }
  return static_cast<int>(hipGetLastError());
}
