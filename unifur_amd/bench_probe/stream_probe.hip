// stream_probe.hip -- streaming kernels that measure what this part moves for
// a given buffer size and read/write mix: the ceilings bench.py sets beside
// the NF4 kernels' roofline fractions.  Measurement only, no counterpart in
// the reference; built as its own library (libunifur_bench_probe.so), not
// part of libunifur_nf4.so or its header.
//
// All are grid-stride loops of 16-byte accesses, four in flight per thread.
// The read folds what it loads into an XOR that it stores only when it
// equals a value the caller passes (never, for the caller's data), so the
// loads cannot be dropped and the only writes are the copy's own.  The mixed
// kernel writes n_write units and reads one source unit per `ratio` of them
// (the source unit i / ratio, so the reads are n_write / ratio units): the
// read/write mix of the dequantize, 8.9 MB read for 67 MB written at 4096^2.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

__global__ __launch_bounds__(kProbeThreads) void stream_mixed_kernel(const u32x4* __restrict__ src, size_t n_read16,
                                                                     uint32_t ratio, u32x4* __restrict__ dst) {
  // a block's 256 source units i0 .. i0 + 255 fan out to its own ratio x 256
  // destination units, written as ratio runs of 4 KiB (each store instruction
  // a contiguous 1 KiB per wave); loads issued a step ahead
  const size_t stride = (size_t)gridDim.x * kProbeThreads;
  size_t i = (size_t)blockIdx.x * kProbeThreads + threadIdx.x;
  u32x4 v = i < n_read16 ? src[i] : u32x4{0u, 0u, 0u, 0u};
  for (; i < n_read16; i += stride) {
    const size_t nx = i + stride;
    const u32x4 next = nx < n_read16 ? src[nx] : u32x4{0u, 0u, 0u, 0u};
    u32x4* d = dst + (i - threadIdx.x) * ratio + threadIdx.x;
    for (uint32_t u = 0; u < ratio; ++u) d[(size_t)u * kProbeThreads] = v ^ u;
    v = next;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

// `bytes` (a multiple of 16) from src over `workgroups` workgroups: a read
// (dst == NULL; sink, 64 u32, is written only if the data XOR to a fixed odd
// value) or a copy to dst.  Returns 0, or -1 for bad arguments, or the HIP
// error code.
int unifur_bench_stream_probe(const void* src, uint64_t bytes, void* dst, uint32_t* sink, uint32_t workgroups,
                              void* stream) {
  if (bytes == 0) return 0;
  if (!src || !sink || bytes % 16 || !aligned16(src) || !aligned16(dst) || workgroups < 1 || workgroups > 65536)
    return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dst)
    stream_copy_kernel<<<workgroups, kProbeThreads, 0, st>>>(static_cast<const u32x4*>(src), bytes / 16,
                                                             static_cast<u32x4*>(dst));
  else
    stream_read_kernel<<<workgroups, kProbeThreads, 0, st>>>(static_cast<const u32x4*>(src), bytes / 16, 0x9e3779b9u,
                                                             sink);
  return (int)hipGetLastError();
}

// Writes `write_bytes` to dst while reading write_bytes / ratio from src;
// write_bytes a multiple of 16 * ratio * 256 (whole blocks).
int unifur_bench_stream_mixed(const void* src, void* dst, uint64_t write_bytes, uint32_t ratio, uint32_t workgroups,
                              void* stream) {
  if (write_bytes == 0) return 0;
  if (!src || !dst || write_bytes % 16 || ratio < 1 || !aligned16(src) || !aligned16(dst) || workgroups < 1 ||
      workgroups > 65536)
    return -1;
  if (write_bytes % (16ull * ratio * kProbeThreads)) return -1;  // whole 256-unit blocks
  stream_mixed_kernel<<<workgroups, kProbeThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(src), write_bytes / 16 / ratio, ratio, static_cast<u32x4*>(dst));
  return (int)hipGetLastError();
}

}  // extern "C"
