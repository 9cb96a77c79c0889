// nf4_generic.hip -- shape-general pieces of the linear path.
//
//   * gemm_f32: Y = X W (+ bias, + LoRA) with W an f32 [d_in, d_out] weight
//     that dequantize() has just written (bit-identical to the reference's
//     dequantized weight).  This is Nf4Linear::forward exactly as the
//     reference runs it -- dequantize, then an f32 matmul
//     (src/qwennet.rs:238-241) -- and serves every shape or precision the
//     fused kernels do not: d_out not a multiple of 64, misaligned buffers,
//     f32 activations with more than four rows.
//   * lora_xa: xa = X A, the first factor of LoraAdapter::forward
//     (src/quantize.rs:619-624); the second factor and the scaling are
//     applied in the consuming kernel's epilogue.
//   * silu_mul: h = silu(g) * u, the middle of QwenMlp::forward
//     (src/qwennet.rs:816-819) when gate and up ran as separate launches;
//     the bf16 variant feeds the MFMA GEMM of the down projection.
#include "nf4_generic.hpp"

namespace unifur {
namespace {

constexpr int kBM = 64, kBN = 64, kBK = 16;

template <bool XBF16>
__device__ __forceinline__ float load_act(const void* x, size_t idx) {
  if constexpr (XBF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(x)[idx]);
  return reinterpret_cast<const float*>(x)[idx];
}

__device__ __forceinline__ float epilogue(const Epilogue& e, float acc, int row, int col, int N) {
  float y = acc;
  if (e.bias) y += e.bias[col];
  if (e.lora_xa) {
    float l = 0.0f;
    for (int j = 0; j < e.lora_rank; ++j)
      l = __builtin_fmaf(e.lora_xa[(size_t)row * e.lora_rank + j], e.lora_b[(size_t)j * N + col], l);
    y += l * e.lora_scaling;
  }
  return y;
}

__device__ __forceinline__ void store_out(const Epilogue& e, size_t idx, float y) {
  if (e.y_bf16)
    reinterpret_cast<uint16_t*>(e.y)[idx] = (uint16_t)(pack_bf16x2(y, 0.0f) & 0xffffu);
  else
    reinterpret_cast<float*>(e.y)[idx] = y;
}

// 64x64 output tile per 256-thread workgroup, 4x4 per thread, K in steps of 16.
template <bool XBF16>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const void* __restrict__ x, const float* __restrict__ w,
                                                       int M, int K, int N, Epilogue e) {
  __shared__ float As[kBK][kBM + 4];
  __shared__ float Bs[kBK][kBN + 4];
  const int tid = threadIdx.x;
  const int tx = tid % 16, ty = tid / 16;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += kBK) {
    for (int i = tid; i < kBM * kBK; i += 256) {
      const int mm = i / kBK, kk = i % kBK;
      const int gm = m0 + mm, gk = k0 + kk;
      As[kk][mm] = (gm < M && gk < K) ? load_act<XBF16>(x, (size_t)gm * K + gk) : 0.0f;
    }
    for (int i = tid; i < kBK * kBN; i += 256) {
      const int kk = i / kBN, nn = i % kBN;
      const int gk = k0 + kk, gn = n0 + nn;
      Bs[kk][nn] = (gk < K && gn < N) ? w[(size_t)gk * N + gn] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gm = m0 + ty * 4 + i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + tx * 4 + j;
      if (gn < N) store_out(e, (size_t)gm * N + gn, epilogue(e, acc[i][j], gm, gn, N));
    }
  }
}

// xa[m][j] = sum_k x[m][k] a[k][j]; 8 rows per workgroup, rank <= 64.
constexpr int kXaRows = 8;
template <bool XBF16>
__global__ __launch_bounds__(256) void lora_xa_kernel(const void* __restrict__ x, const float* __restrict__ a, int M,
                                                      int K, int rank, float* __restrict__ xa) {
  const int m0 = blockIdx.x * kXaRows;
  const int tid = threadIdx.x;
  // thread owns (row m0 + tid / 32, rank column tid % 32, +32) over all k
  const int rr = tid / 32, jj = tid % 32;
  const int m = m0 + rr;
  float acc0 = 0.0f, acc1 = 0.0f;
  if (m < M) {
    for (int k = 0; k < K; ++k) {
      const float xv = load_act<XBF16>(x, (size_t)m * K + k);
      if (jj < rank) acc0 = __builtin_fmaf(xv, a[(size_t)k * rank + jj], acc0);
      if (jj + 32 < rank) acc1 = __builtin_fmaf(xv, a[(size_t)k * rank + jj + 32], acc1);
    }
    if (jj < rank) xa[(size_t)m * rank + jj] = acc0;
    if (jj + 32 < rank) xa[(size_t)m * rank + jj + 32] = acc1;
  }
}

__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, size_t n,
                                float* __restrict__ h) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float z = g[i];
    h[i] = (z * (1.0f / (1.0f + __expf(-z)))) * u[i];
  }
}

__global__ void silu_mul_bf16_kernel(const float* __restrict__ g, const float* __restrict__ u, size_t n,
                                     uint16_t* __restrict__ h) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float z = g[i];
    h[i] = (uint16_t)(pack_bf16x2((z * (1.0f / (1.0f + __expf(-z)))) * u[i], 0.0f) & 0xffffu);
  }
}

// out[k][n] = w[k][n] + (sum_j a[k][j] b[j][n]) * scaling: QLoraLinear::merged
// (src/quantize.rs:716-726) with LoraAdapter::delta_weight (src/quantize.rs:626-634)
// evaluated in that order (product, then the scale, then the sum).
__global__ void lora_merge_kernel(const float* __restrict__ w, const float* __restrict__ a,
                                  const float* __restrict__ b, int rank, float scaling, uint64_t K, uint64_t N,
                                  float* __restrict__ out) {
  const uint64_t total = K * N;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t k = i / N, n = i % N;
    float d = 0.0f;
    for (int j = 0; j < rank; ++j) d = __builtin_fmaf(a[k * rank + j], b[(uint64_t)j * N + n], d);
    out[i] = w[i] + d * scaling;
  }
}

}  // namespace

hipError_t launch_lora_merge(const float* w, const float* a, const float* b, int rank, float scaling, uint64_t K,
                             uint64_t N, float* out, hipStream_t stream) {
  const uint64_t total = K * N;
  if (total == 0) return hipSuccess;
  uint64_t blocks = (total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  lora_merge_kernel<<<(unsigned)blocks, 256, 0, stream>>>(w, a, b, rank, scaling, K, N, out);
  return hipGetLastError();
}

hipError_t launch_gemm_f32(const void* x, bool x_bf16, const float* w, int M, int K, int N, const Epilogue& e,
                           hipStream_t stream) {
  dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
  if (x_bf16)
    gemm_f32_kernel<true><<<grid, 256, 0, stream>>>(x, w, M, K, N, e);
  else
    gemm_f32_kernel<false><<<grid, 256, 0, stream>>>(x, w, M, K, N, e);
  return hipGetLastError();
}

hipError_t launch_lora_xa(const void* x, bool x_bf16, const float* a, int M, int K, int rank, float* xa,
                          hipStream_t stream) {
  if (rank > 64) return hipErrorInvalidValue;
  const int grid = (M + kXaRows - 1) / kXaRows;
  if (x_bf16)
    lora_xa_kernel<true><<<grid, 256, 0, stream>>>(x, a, M, K, rank, xa);
  else
    lora_xa_kernel<false><<<grid, 256, 0, stream>>>(x, a, M, K, rank, xa);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const float* g, const float* u, size_t n, float* h, hipStream_t stream) {
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks == 0) return hipSuccess;
  silu_mul_kernel<<<(unsigned)blocks, 256, 0, stream>>>(g, u, n, h);
  return hipGetLastError();
}

hipError_t launch_silu_mul_bf16(const float* g, const float* u, size_t n, uint16_t* h, hipStream_t stream) {
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks == 0) return hipSuccess;
  silu_mul_bf16_kernel<<<(unsigned)blocks, 256, 0, stream>>>(g, u, n, h);
  return hipGetLastError();
}

}  // namespace unifur
