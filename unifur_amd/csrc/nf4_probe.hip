// nf4_probe.hip -- streaming read / copy kernels that measure what this part
// streams for a given buffer size (the ceiling the decode GEMV's roofline
// fraction is compared with).  No counterpart in the reference.
//
// Both are grid-stride loops of 16-byte accesses, four in flight per thread;
// the read folds what it loads into an XOR that it stores only when it
// equals a value the caller passes (never, for the caller's data), so the
// loads cannot be dropped and the only writes are the copy's own.
#include "nf4_probe.hpp"

namespace unifur {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;

__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4* __restrict__ src, size_t n16,
                                                                    uint32_t never, uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * kProbeThreads;
  size_t i = (size_t)blockIdx.x * kProbeThreads + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= src[i];
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == never) sink[blockIdx.x & 63] = x;
}

__global__ __launch_bounds__(kProbeThreads) void stream_copy_kernel(const u32x4* __restrict__ src, size_t n16,
                                                                    u32x4* __restrict__ dst) {
  const size_t stride = (size_t)gridDim.x * kProbeThreads;
  size_t i = (size_t)blockIdx.x * kProbeThreads + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) dst[i + u * stride] = v[u];
  }
  for (; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace

hipError_t launch_stream_probe(const void* src, size_t n16, void* dst, uint32_t never, uint32_t* sink, int grid,
                               hipStream_t stream) {
  if (n16 == 0) return hipSuccess;
  if (dst)
    stream_copy_kernel<<<grid, kProbeThreads, 0, stream>>>(static_cast<const u32x4*>(src), n16,
                                                           static_cast<u32x4*>(dst));
  else
    stream_read_kernel<<<grid, kProbeThreads, 0, stream>>>(static_cast<const u32x4*>(src), n16, never, sink);
  return hipGetLastError();
}

}  // namespace unifur
