// nf4_expand.hpp -- NF4 weight -> bf16 GEMM operand, and the BLAS GEMM that
// consumes it (the prefill path for batches above the skinny kernel's).
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

// K and N multiples of 64, rank <= 64.
bool expand_supported(int K, int N, int rank);

// Wt[N][K] bf16 = the dequantized weight (row-major or striped layout) plus
// scaling * A B when rank > 0 (A f32 [K][rank], B f32 [rank][N], read by the
// kernel itself and rounded to bf16 for its MFMAs).
hipError_t launch_expand_bf16(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                              const float* lora_a, const float* lora_b, int rank, float scaling, uint16_t* wt,
                              hipStream_t stream);
// The columns [n_begin, n_end) (multiples of 64) of Wt only.
hipError_t launch_expand_cols(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                              const float* lora_a, const float* lora_b, int rank, float scaling, int n_begin, int n_end,
                              uint16_t* wt, hipStream_t stream);

// E[K][N] bf16 row-major (the weight's own orientation): the same values as
// launch_expand_bf16 writes transposed, rank 0 included.  The backward's
// dX = dY E^T then runs as blas_gemm_xwt, the forward's TN product.
hipError_t launch_expand_rows_bf16(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                                   const float* lora_a, const float* lora_b, int rank, float scaling, uint16_t* e,
                                   hipStream_t stream);

// Scratch the BLAS GEMM may use (its kernels' split-K partials and the like).
constexpr size_t kBlasWorkspace = 32u << 20;

// Y[M][N] = X[M][K] Wt[N][K]^T (+ bias[N]): bf16 operands, f32 accumulation,
// Y f32 or bf16, row-major, through hipBLASLt.  The kernel for a shape is
// chosen on its first call on a device by timing the library's candidates on
// `stream` (a host wait); a first call under stream capture takes the
// library's first candidate without caching it.
hipError_t blas_gemm_xwt(const uint16_t* x, const uint16_t* wt, const float* bias, int M, int N, int K, void* y,
                         bool y_bf16, void* ws, size_t ws_bytes, hipStream_t stream);
// The same product into columns of a wider Y (row stride ldy >= N elements).
hipError_t blas_gemm_xwt_ld(const uint16_t* x, const uint16_t* wt, const float* bias, int M, int N, int K, void* y,
                            int ldy, bool y_bf16, void* ws, size_t ws_bytes, hipStream_t stream);

// Whether this device has chosen its blas_gemm_xwt kernel for the shape
// (without bias; a call before that times the candidates, which wants the
// GPU to itself).
bool blas_gemm_xwt_tuned(int M, int N, int K, bool y_bf16);

}  // namespace unifur
