// nf4_layout.hip -- the column-striped device layout of a linear weight.
//
// The reference stores an Nf4Linear weight as the packed codes of its
// [d_in, d_out] row-major values (src/qwennet.rs:161-205, blocks of 64 along
// d_out) with per-block scales in the same flat order.  For the decode GEMV
// every workgroup wants a narrow column band over the whole of d_in, which
// that order scatters across d_in rows d_out/2 bytes apart.  The striped
// layout is a pure byte permutation of the same data (so it round-trips bit
// for bit and has the same size):
//
//   codes:  16-column stripe s (8 bytes of one row) of all K rows contiguous,
//           striped[(s * K + k) * 8 + j] = row_major[k * N / 2 + s * 8 + j]
//   scales: block-major, striped[b * K + k] = row_major[k * N / 64 + b]
//
// with K = d_in, N = d_out (a multiple of 64).  Both are transposes of small
// fixed-size elements (u64 code groups, u8 or f32 scales), done here with a
// 64 x 64 tile staged through LDS so that reads and writes are coalesced.
#include "nf4_layout.hpp"

namespace unifur {
namespace {

constexpr int kTile = 64;

// dst[c][r] = src[r][c] for a rows x cols matrix of T.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, uint64_t rows,
                                                        uint64_t cols) {
  __shared__ T tile[kTile][kTile + 1];
  const int tid = threadIdx.x;
  const uint64_t r0 = (uint64_t)blockIdx.y * kTile, c0 = (uint64_t)blockIdx.x * kTile;
  const int lc = tid & 63, lr = tid >> 6;
#pragma unroll
  for (int i = 0; i < kTile / 4; ++i) {
    const int r = lr + 4 * i;
    if (r0 + r < rows && c0 + lc < cols) tile[r][lc] = src[(r0 + r) * cols + c0 + lc];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile / 4; ++i) {
    const int c = lr + 4 * i;
    if (c0 + c < cols && r0 + lc < rows) dst[(c0 + c) * rows + r0 + lc] = tile[lc][c];
  }
}

template <typename T>
hipError_t launch_transpose(const void* src, void* dst, uint64_t rows, uint64_t cols, hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const uint64_t gx = (cols + kTile - 1) / kTile, gy = (rows + kTile - 1) / kTile;
  if (gx > 0x7fffffffu || gy > 65535u) return hipErrorInvalidValue;
  transpose_kernel<T><<<dim3((unsigned)gx, (unsigned)gy), 256, 0, stream>>>(static_cast<const T*>(src),
                                                                            static_cast<T*>(dst), rows, cols);
  return hipGetLastError();
}

// dst[c][r] = decode(src[r][c]) into f32: the checkpoint's [out, in]
// weight (f32, or bf16 / f16 decoded exactly) to the [in, out] f32 values
// that quantize takes.
template <int SRC>
__global__ __launch_bounds__(256) void transpose_decode_kernel(const void* __restrict__ src, float* __restrict__ dst,
                                                               uint64_t rows, uint64_t cols) {
  __shared__ float tile[kTile][kTile + 1];
  const int tid = threadIdx.x;
  const uint64_t r0 = (uint64_t)blockIdx.y * kTile, c0 = (uint64_t)blockIdx.x * kTile;
  const int lc = tid & 63, lr = tid >> 6;
#pragma unroll
  for (int i = 0; i < kTile / 4; ++i) {
    const int r = lr + 4 * i;
    if (r0 + r < rows && c0 + lc < cols) {
      const uint64_t idx = (r0 + r) * cols + c0 + lc;
      tile[r][lc] = decode_src<SRC>(src, idx);
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile / 4; ++i) {
    const int c = lr + 4 * i;
    if (c0 + c < cols && r0 + lc < rows) dst[(c0 + c) * rows + r0 + lc] = tile[lc][c];
  }
}

}  // namespace

hipError_t launch_transpose_decode(const void* src, int src_kind, uint64_t rows, uint64_t cols, float* dst,
                                   hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const uint64_t gx = (cols + kTile - 1) / kTile, gy = (rows + kTile - 1) / kTile;
  if (gx > 0x7fffffffu || gy > 65535u) return hipErrorInvalidValue;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  switch (src_kind) {
    case kSrcF32: transpose_decode_kernel<kSrcF32><<<grid, 256, 0, stream>>>(src, dst, rows, cols); break;
    case kSrcBf16: transpose_decode_kernel<kSrcBf16><<<grid, 256, 0, stream>>>(src, dst, rows, cols); break;
    case kSrcF16: transpose_decode_kernel<kSrcF16><<<grid, 256, 0, stream>>>(src, dst, rows, cols); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_stripe_codes(const uint8_t* src, uint8_t* dst, uint64_t d_in, uint64_t d_out, bool to_striped,
                               hipStream_t stream) {
  // codes as a [d_in, d_out / 16] matrix of u64 groups (row-major), or its
  // transpose [d_out / 16, d_in] (striped)
  const uint64_t groups = d_out / kStripeCols;
  if (to_striped) return launch_transpose<uint64_t>(src, dst, d_in, groups, stream);
  return launch_transpose<uint64_t>(src, dst, groups, d_in, stream);
}

hipError_t launch_stripe_scales(const void* src, void* dst, uint64_t d_in, uint64_t d_out, bool dq, bool to_striped,
                                hipStream_t stream) {
  // [d_in, d_out / 64] (row-major) or [d_out / 64, d_in] (striped)
  const uint64_t blocks = d_out / kBlock;
  const uint64_t rows = to_striped ? d_in : blocks, cols = to_striped ? blocks : d_in;
  if (dq) return launch_transpose<uint8_t>(src, dst, rows, cols, stream);
  return launch_transpose<float>(src, dst, rows, cols, stream);
}

}  // namespace unifur
