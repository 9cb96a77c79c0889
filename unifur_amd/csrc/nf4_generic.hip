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
//   * backward pieces (the autodiff of the two forwards above with the
//     base weight frozen): gemm_f32 with the weight read transposed
//     (dX = dY W^T), lora_xa with strided factors (dY B^T), and row_atb,
//     C = scale * P^T Q summed over the rows in a fixed order (the adapter
//     gradients).
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

// 64x64 output tile per 256-thread workgroup, 4x4 per thread, K in steps of
// 16; w is [K, N] row-major, or with WT its transpose stored [N, K].
template <bool XBF16, bool WT>
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
      Bs[kk][nn] = (gk < K && gn < N) ? (WT ? w[(size_t)gn * K + gk] : w[(size_t)gk * N + gn]) : 0.0f;
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
                                                      int K, int rank, size_t sk, size_t sj, float* __restrict__ xa) {
  const int m0 = blockIdx.x * kXaRows;
  const int tid = threadIdx.x;
  // thread owns (row m0 + tid / 32, rank column tid % 32, +32) over all k
  const int rr = tid / 32, jj = tid % 32;
  const int m = m0 + rr;
  float acc0 = 0.0f, acc1 = 0.0f;
  if (m < M) {
    for (int k = 0; k < K; ++k) {
      const float xv = load_act<XBF16>(x, (size_t)m * K + k);
      if (jj < rank) acc0 = __builtin_fmaf(xv, a[(size_t)k * sk + (size_t)jj * sj], acc0);
      if (jj + 32 < rank) acc1 = __builtin_fmaf(xv, a[(size_t)k * sk + (size_t)(jj + 32) * sj], acc1);
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

// h[m][i] = bf16(silu(g) * u) with g = gu[m][i] and u = gu[m][inter + i]
// (the gate and up halves of one GEMM's output row), gu f32 or bf16.
__device__ __forceinline__ float gu_value(const uint16_t* p, size_t i) { return bf16_bits_to_f32(p[i]); }
__device__ __forceinline__ float gu_value(const float* p, size_t i) { return p[i]; }

template <typename TIn>
__global__ void silu_mul_rows_bf16_kernel(const TIn* __restrict__ gu, size_t rows, size_t inter,
                                          uint16_t* __restrict__ h) {
  const size_t n = rows * inter;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const size_t m = i / inter, c = i % inter;
    const float z = gu_value(gu, m * 2 * inter + c);
    const float u = gu_value(gu, m * 2 * inter + inter + c);
    h[i] = (uint16_t)(pack_bf16x2((z * (1.0f / (1.0f + __expf(-z)))) * u, 0.0f) & 0xffffu);
  }
}

// The same for bf16 gu, inter % 8 == 0 and 16-byte aligned buffers: eight
// values per thread, two 16-byte loads and one 16-byte store; n8 = rows *
// inter / 8 and the row arithmetic fit 32 bits.
__global__ __launch_bounds__(256) void silu_mul_rows_bf16_v8_kernel(const uint16_t* __restrict__ gu, uint32_t inter8,
                                                                    uint32_t n8, uint16_t* __restrict__ h) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += gridDim.x * blockDim.x) {
    const uint32_t m = i / inter8, c8 = i - m * inter8;
    const size_t row = (size_t)m * inter8 * 16;  // 2 inter values per gu row
    const u32x4 gz = *reinterpret_cast<const u32x4*>(gu + row + (size_t)c8 * 8);
    const u32x4 gv = *reinterpret_cast<const u32x4*>(gu + row + (size_t)inter8 * 8 + (size_t)c8 * 8);
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float r[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float z = bf16_bits_to_f32(e ? gz[k] >> 16 : gz[k] & 0xffffu);
        const float u = bf16_bits_to_f32(e ? gv[k] >> 16 : gv[k] & 0xffffu);
        r[e] = (z * (1.0f / (1.0f + __expf(-z)))) * u;
      }
      o[k] = pack_bf16x2(r[0], r[1]);
    }
    *reinterpret_cast<u32x4*>(h + (size_t)i * 8) = o;
  }
}

__global__ void silu_mul_bf16_kernel(const float* __restrict__ g, const float* __restrict__ u, size_t n,
                                     uint16_t* __restrict__ h) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float z = g[i];
    h[i] = (uint16_t)(pack_bf16x2((z * (1.0f / (1.0f + __expf(-z)))) * u[i], 0.0f) & 0xffffu);
  }
}

// partials[s][i][j] = sum over the rows of slab s of p[m][i] q[m][j]: the
// gemm_f32 tiling with the contraction over rows; 64 x 64 tile of (i, j)
// per workgroup, slab s = blockIdx.z covers rows [s rows, (s + 1) rows).
template <bool PBF16, bool QBF16>
__global__ __launch_bounds__(256) void row_atb_kernel(const void* __restrict__ p, const void* __restrict__ q, int M,
                                                      int P, int Q, int rows, float* __restrict__ partials) {
  __shared__ float Ps[kBK][kBM + 4];
  __shared__ float Qs[kBK][kBN + 4];
  const int tid = threadIdx.x;
  const int tx = tid % 16, ty = tid / 16;
  const int i0 = blockIdx.y * kBM, j0 = blockIdx.x * kBN;
  const int mb = blockIdx.z * rows, me = min(M, mb + rows);
  float acc[4][4] = {};
  for (int m0 = mb; m0 < me; m0 += kBK) {
    for (int t = tid; t < kBK * kBM; t += 256) {
      const int mm = t / kBM, ii = t % kBM;
      const int gm = m0 + mm, gi = i0 + ii;
      Ps[mm][ii] = (gm < me && gi < P) ? load_act<PBF16>(p, (size_t)gm * P + gi) : 0.0f;
    }
    for (int t = tid; t < kBK * kBN; t += 256) {
      const int mm = t / kBN, jj = t % kBN;
      const int gm = m0 + mm, gj = j0 + jj;
      Qs[mm][jj] = (gm < me && gj < Q) ? load_act<QBF16>(q, (size_t)gm * Q + gj) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int mm = 0; mm < kBK; ++mm) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = Ps[mm][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Qs[mm][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  float* out = partials + (size_t)blockIdx.z * P * Q;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gi = i0 + ty * 4 + i;
    if (gi >= P) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gj = j0 + tx * 4 + j;
      if (gj < Q) out[(size_t)gi * Q + gj] = acc[i][j];
    }
  }
}

// c[i] = scale * (partials[0][i] + partials[1][i] + ...), slabs in order.
__global__ void slab_sum_kernel(const float* __restrict__ partials, int slabs, size_t n, float scale,
                                float* __restrict__ c) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    float sum = 0.0f;
    for (int s = 0; s < slabs; ++s) sum += partials[(size_t)s * n + i];
    c[i] = sum * scale;
  }
}

// Narrow products of the adapter backward, over slabs into partials that
// slab_sum_kernel adds in a fixed order.
//
// narrow_mm: partials[s][m][j] = sum over the K slab s of x[m][k] w(k, j),
// j < R <= 64, w(k, j) = w[k][j] (w [K][R]) or, with WT, w[j][k] (w [R][K]).
// 64 rows x R per workgroup; thread t owns row t / 4 and columns
// (t % 4) R / 4 .. + R / 4 - 1; x and w tiles of 16 k staged in LDS.
template <bool XBF16, bool WT, int R>
__global__ __launch_bounds__(256) void narrow_mm_kernel(const void* __restrict__ x, const float* __restrict__ w,
                                                        int M, int K, int rank, int kslab,
                                                        float* __restrict__ partials) {
  constexpr int C = R / 4;
  __shared__ float Xs[kBK][64 + 1];
  __shared__ float Ws[kBK][R];
  const int tid = threadIdx.x;
  const int row = tid >> 2, jq = tid & 3;
  const int m0 = blockIdx.x * 64;
  const int kb = blockIdx.y * kslab, ke = min(K, kb + kslab);
  float acc[C] = {};
  for (int k0 = kb; k0 < ke; k0 += kBK) {
    for (int i = tid; i < 64 * kBK; i += 256) {
      const int mm = i / kBK, kk = i % kBK;
      const int gm = m0 + mm, gk = k0 + kk;
      Xs[kk][mm] = (gm < M && gk < ke) ? load_act<XBF16>(x, (size_t)gm * K + gk) : 0.0f;
    }
    for (int i = tid; i < kBK * R; i += 256) {
      const int kk = i / R, j = i % R;
      const int gk = k0 + kk;
      Ws[kk][j] = (gk < ke && j < rank) ? (WT ? w[(size_t)j * K + gk] : w[(size_t)gk * rank + j]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      const float xv = Xs[kk][row];
#pragma unroll
      for (int c = 0; c < C; ++c) acc[c] = __builtin_fmaf(xv, Ws[kk][jq * C + c], acc[c]);
    }
    __syncthreads();
  }
  const int gm = m0 + row;
  if (gm < M) {
    float* out = partials + ((size_t)blockIdx.y * M + gm) * rank;
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (jq * C + c < rank) out[jq * C + c] = acc[c];
  }
}

// narrow_atb: partials[s] of sum over the rows m of slab s of
// wide[m][v] nar[m][j] (v < W, j < R <= 64), stored [v][j] or, with
// NAR_MAJOR, [j][v].  256 wide indices x R per workgroup: thread t owns
// v = 256 blockIdx.x + t and all R sums; the narrow rows are staged in LDS
// 16 at a time and read as broadcasts.
template <bool WBF16, bool NAR_MAJOR, int R>
__global__ __launch_bounds__(256) void narrow_atb_kernel(const void* __restrict__ wide, const float* __restrict__ nar,
                                                         int M, int W, int rank, int mslab,
                                                         float* __restrict__ partials) {
  __shared__ float Ns[kBK][R];
  const int tid = threadIdx.x;
  const int v = blockIdx.x * 256 + tid;
  const int mb = blockIdx.y * mslab, me = min(M, mb + mslab);
  float acc[R] = {};
  for (int m0 = mb; m0 < me; m0 += kBK) {
    for (int i = tid; i < kBK * R; i += 256) {
      const int mm = i / R, j = i % R;
      Ns[mm][j] = (m0 + mm < me && j < rank) ? nar[(size_t)(m0 + mm) * rank + j] : 0.0f;
    }
    __syncthreads();
    const int mn = min(kBK, me - m0);
    if (v < W) {
      for (int mm = 0; mm < mn; ++mm) {
        const float wv = load_act<WBF16>(wide, (size_t)(m0 + mm) * W + v);
#pragma unroll
        for (int j = 0; j < R; ++j) acc[j] = __builtin_fmaf(wv, Ns[mm][j], acc[j]);
      }
    }
    __syncthreads();
  }
  if (v < W) {
    float* out = partials + (size_t)blockIdx.y * W * rank;
#pragma unroll
    for (int j = 0; j < R; ++j)
      if (j < rank) out[NAR_MAJOR ? (size_t)j * W + v : (size_t)v * rank + j] = acc[j];
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
    gemm_f32_kernel<true, false><<<grid, 256, 0, stream>>>(x, w, M, K, N, e);
  else
    gemm_f32_kernel<false, false><<<grid, 256, 0, stream>>>(x, w, M, K, N, e);
  return hipGetLastError();
}

hipError_t launch_gemm_f32_wt(const void* x, bool x_bf16, const float* wt, int M, int K, int N, const Epilogue& e,
                              hipStream_t stream) {
  dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
  if (x_bf16)
    gemm_f32_kernel<true, true><<<grid, 256, 0, stream>>>(x, wt, M, K, N, e);
  else
    gemm_f32_kernel<false, true><<<grid, 256, 0, stream>>>(x, wt, M, K, N, e);
  return hipGetLastError();
}

hipError_t launch_lora_xa_strided(const void* x, bool x_bf16, const float* a, size_t sk, size_t sj, int M, int K,
                                  int rank, float* xa, hipStream_t stream) {
  if (rank > 64) return hipErrorInvalidValue;
  const int grid = (M + kXaRows - 1) / kXaRows;
  if (x_bf16)
    lora_xa_kernel<true><<<grid, 256, 0, stream>>>(x, a, M, K, rank, sk, sj, xa);
  else
    lora_xa_kernel<false><<<grid, 256, 0, stream>>>(x, a, M, K, rank, sk, sj, xa);
  return hipGetLastError();
}

hipError_t launch_lora_xa(const void* x, bool x_bf16, const float* a, int M, int K, int rank, float* xa,
                          hipStream_t stream) {
  return launch_lora_xa_strided(x, x_bf16, a, (size_t)rank, 1, M, K, rank, xa, stream);
}

int row_atb_slabs(int M, int P, int Q) {
  const int tiles = P > 0 && Q > 0 ? ((P + kBM - 1) / kBM) * ((Q + kBN - 1) / kBN) : 1;
  int slabs = (512 + tiles - 1) / tiles;
  const int max_slabs = (M + kBK - 1) / kBK;
  if (slabs > max_slabs) slabs = max_slabs;
  if (slabs > 64) slabs = 64;
  return slabs < 1 ? 1 : slabs;
}

hipError_t launch_row_atb(const void* p, bool p_bf16, const void* q, bool q_bf16, int M, int P, int Q, float scale,
                          float* partials, float* c, hipStream_t stream) {
  if (M < 0 || P <= 0 || Q <= 0) return hipSuccess;  // M == 0 still writes the zero sums
  const int slabs = row_atb_slabs(M, P, Q);
  const int rows = ((M + slabs - 1) / slabs + kBK - 1) / kBK * kBK;
  dim3 grid((Q + kBN - 1) / kBN, (P + kBM - 1) / kBM, slabs);
  if (p_bf16) {
    if (q_bf16) row_atb_kernel<true, true><<<grid, 256, 0, stream>>>(p, q, M, P, Q, rows, partials);
    else row_atb_kernel<true, false><<<grid, 256, 0, stream>>>(p, q, M, P, Q, rows, partials);
  } else {
    if (q_bf16) row_atb_kernel<false, true><<<grid, 256, 0, stream>>>(p, q, M, P, Q, rows, partials);
    else row_atb_kernel<false, false><<<grid, 256, 0, stream>>>(p, q, M, P, Q, rows, partials);
  }
  const size_t n = (size_t)P * Q;
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  slab_sum_kernel<<<(unsigned)blocks, 256, 0, stream>>>(partials, slabs, n, scale, c);
  return hipGetLastError();
}

namespace {

int narrow_bucket(int rank) { return rank <= 16 ? 16 : rank <= 32 ? 32 : 64; }

hipError_t slab_sum(const float* partials, int slabs, size_t n, float scale, float* out, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  slab_sum_kernel<<<(unsigned)blocks, 256, 0, stream>>>(partials, slabs, n, scale, out);
  return hipGetLastError();
}

}  // namespace

int narrow_mm_slabs(int M, int K) {
  const int tiles = M > 0 ? (M + 63) / 64 : 1;
  int slabs = (512 + tiles - 1) / tiles;
  const int max_slabs = (K + kBK - 1) / kBK;
  if (slabs > max_slabs) slabs = max_slabs;
  if (slabs > 64) slabs = 64;
  return slabs < 1 ? 1 : slabs;
}

hipError_t launch_narrow_mm(const void* x, bool x_bf16, const float* w, bool w_t, int M, int K, int rank,
                            float* partials, float* out, hipStream_t stream) {
  if (M <= 0 || rank <= 0 || rank > 64) return M == 0 ? hipSuccess : hipErrorInvalidValue;
  const int slabs = narrow_mm_slabs(M, K);
  const int kslab = ((K + slabs - 1) / slabs + kBK - 1) / kBK * kBK;
  dim3 grid((M + 63) / 64, slabs);
#define UNIFUR_NMM(XB, WT, R) narrow_mm_kernel<XB, WT, R><<<grid, 256, 0, stream>>>(x, w, M, K, rank, kslab, partials)
#define UNIFUR_NMM_R(XB, WT)                  \
  do {                                        \
    const int b_ = narrow_bucket(rank);       \
    if (b_ == 16) UNIFUR_NMM(XB, WT, 16);     \
    else if (b_ == 32) UNIFUR_NMM(XB, WT, 32); \
    else UNIFUR_NMM(XB, WT, 64);              \
  } while (0)
  if (x_bf16) {
    if (w_t) UNIFUR_NMM_R(true, true); else UNIFUR_NMM_R(true, false);
  } else {
    if (w_t) UNIFUR_NMM_R(false, true); else UNIFUR_NMM_R(false, false);
  }
#undef UNIFUR_NMM_R
#undef UNIFUR_NMM
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return slab_sum(partials, slabs, (size_t)M * rank, 1.0f, out, stream);
}

int narrow_atb_slabs(int M, int W) {
  const int tiles = W > 0 ? (W + 255) / 256 : 1;
  int slabs = (512 + tiles - 1) / tiles;
  const int max_slabs = (M + kBK - 1) / kBK;
  if (slabs > max_slabs) slabs = max_slabs;
  if (slabs > 64) slabs = 64;
  return slabs < 1 ? 1 : slabs;
}

hipError_t launch_narrow_atb(const void* wide, bool wide_bf16, const float* nar, int M, int W, int rank,
                             bool nar_major, float scale, float* partials, float* out, hipStream_t stream) {
  if (W <= 0 || rank <= 0 || rank > 64 || M < 0) return hipErrorInvalidValue;
  const int slabs = narrow_atb_slabs(M, W);
  const int mslab = ((M + slabs - 1) / slabs + kBK - 1) / kBK * kBK;
  dim3 grid((W + 255) / 256, slabs);
#define UNIFUR_NATB(WB, NM, R) narrow_atb_kernel<WB, NM, R><<<grid, 256, 0, stream>>>(wide, nar, M, W, rank, mslab, partials)
#define UNIFUR_NATB_R(WB, NM)                 \
  do {                                        \
    const int b_ = narrow_bucket(rank);       \
    if (b_ == 16) UNIFUR_NATB(WB, NM, 16);    \
    else if (b_ == 32) UNIFUR_NATB(WB, NM, 32); \
    else UNIFUR_NATB(WB, NM, 64);             \
  } while (0)
  if (wide_bf16) {
    if (nar_major) UNIFUR_NATB_R(true, true); else UNIFUR_NATB_R(true, false);
  } else {
    if (nar_major) UNIFUR_NATB_R(false, true); else UNIFUR_NATB_R(false, false);
  }
#undef UNIFUR_NATB_R
#undef UNIFUR_NATB
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return slab_sum(partials, slabs, (size_t)W * rank, scale, out, stream);
}

// f32 gu with inter % 4 == 0 and 16-byte aligned buffers: four values per
// thread, two 16-byte loads and one 8-byte store; n4 fits 32 bits.
__global__ __launch_bounds__(256) void silu_mul_rows_f32_v4_kernel(const float* __restrict__ gu, uint32_t inter4,
                                                                   uint32_t n4, uint16_t* __restrict__ h) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
    const uint32_t m = i / inter4, c4 = i - m * inter4;
    const size_t row = (size_t)m * inter4 * 8;  // 2 inter values per gu row
    const f32x4 z4 = *reinterpret_cast<const f32x4*>(gu + row + (size_t)c4 * 4);
    const f32x4 u4 = *reinterpret_cast<const f32x4*>(gu + row + (size_t)inter4 * 4 + (size_t)c4 * 4);
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (z4[e] * (1.0f / (1.0f + __expf(-z4[e])))) * u4[e];
    *reinterpret_cast<u32x2*>(h + (size_t)i * 4) = u32x2{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
  }
}

hipError_t launch_silu_mul_rows_bf16(const void* gu, bool gu_f32, size_t rows, size_t inter, uint16_t* h,
                                     hipStream_t stream) {
  const size_t n = rows * inter;
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks == 0) return hipSuccess;
  if (gu_f32 && inter % 4 == 0 && n / 4 <= 0xffffffffu &&
      ((reinterpret_cast<uintptr_t>(gu) | reinterpret_cast<uintptr_t>(h)) & 15u) == 0) {
    const size_t n4 = n / 4;
    const size_t b4 = std::min<size_t>((n4 + 255) / 256, 16384);
    silu_mul_rows_f32_v4_kernel<<<(unsigned)b4, 256, 0, stream>>>(static_cast<const float*>(gu),
                                                                  (uint32_t)(inter / 4), (uint32_t)n4, h);
    return hipGetLastError();
  }
  if (gu_f32) {
    silu_mul_rows_bf16_kernel<float><<<(unsigned)blocks, 256, 0, stream>>>(static_cast<const float*>(gu), rows, inter,
                                                                           h);
    return hipGetLastError();
  }
  const uint16_t* gb = static_cast<const uint16_t*>(gu);
  const size_t n8 = n / 8;
  if (inter % 8 == 0 && n8 <= 0xffffffffu && ((reinterpret_cast<uintptr_t>(gb) | reinterpret_cast<uintptr_t>(h)) & 15u) == 0) {
    const size_t b8 = std::min<size_t>((n8 + 255) / 256, 16384);
    silu_mul_rows_bf16_v8_kernel<<<(unsigned)b8, 256, 0, stream>>>(gb, (uint32_t)(inter / 8), (uint32_t)n8, h);
    return hipGetLastError();
  }
  silu_mul_rows_bf16_kernel<uint16_t><<<(unsigned)blocks, 256, 0, stream>>>(gb, rows, inter, h);
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

// One workgroup per row: the sum of squares over the row in f32 (threads
// stride the row, then a fixed-order tree), then every element scaled.
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* __restrict__ x, int x_bf16, int h,
                                                       const float* __restrict__ w, float eps, void* __restrict__ out,
                                                       int out_bf16) {
  __shared__ float part[256];
  const size_t row = blockIdx.x;
  const int t = threadIdx.x;
  auto load = [&](int i) -> float {
    return x_bf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(x)[row * h + i])
                  : static_cast<const float*>(x)[row * h + i];
  };
  float ss = 0.0f;
  for (int i = t; i < h; i += 256) {
    const float v = load(i);
    ss = __builtin_fmaf(v, v, ss);
  }
  part[t] = ss;
  __syncthreads();
  for (int m = 128; m > 0; m >>= 1) {
    if (t < m) part[t] += part[t + m];
    __syncthreads();
  }
  const float inv = 1.0f / __builtin_sqrtf(part[0] / (float)h + eps);
  for (int i = t; i < h; i += 256) {
    const float v = (load(i) * inv) * (w[i] + 1.0f);
    if (out_bf16)
      static_cast<uint16_t*>(out)[row * h + i] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
    else
      static_cast<float*>(out)[row * h + i] = v;
  }
}

__global__ __launch_bounds__(256) void add_kernel(const void* __restrict__ a, const void* __restrict__ b, int bf16,
                                                  size_t n, void* __restrict__ y) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    if (bf16) {
      const float v = bf16_bits_to_f32(static_cast<const uint16_t*>(a)[i]) +
                      bf16_bits_to_f32(static_cast<const uint16_t*>(b)[i]);
      static_cast<uint16_t*>(y)[i] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
    } else {
      static_cast<float*>(y)[i] = static_cast<const float*>(a)[i] + static_cast<const float*>(b)[i];
    }
  }
}

hipError_t launch_rms_norm(const void* x, bool x_bf16, int rows, int h, const float* w, float eps, void* out,
                           bool out_bf16, hipStream_t stream) {
  if (rows <= 0 || h <= 0) return hipSuccess;
  rms_norm_kernel<<<(unsigned)rows, 256, 0, stream>>>(x, x_bf16, h, w, eps, out, out_bf16);
  return hipGetLastError();
}

hipError_t launch_add(const void* a, const void* b, bool bf16, size_t n, void* y, hipStream_t stream) {
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks == 0) return hipSuccess;
  add_kernel<<<(unsigned)blocks, 256, 0, stream>>>(a, b, bf16, n, y);
  return hipGetLastError();
}

}  // namespace unifur
