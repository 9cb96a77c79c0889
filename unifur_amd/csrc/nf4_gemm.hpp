// nf4_gemm.hpp -- internal interface of the MFMA prefill GEMM.
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

// Shapes and buffers the MFMA GEMM takes: bf16 X 16-byte aligned, K a
// multiple of 64, N a multiple of 128 (whole 128 x 128 tiles along N; rows
// past M are masked), (M + 256) K bf16 values under 2 GiB (32-bit buffer
// offsets).
bool gemm_supported(int M, int K, int N, const void* x);

// Row stride (in floats) of the xa buffer launch_lora_xa_bf16 writes.
int lora_pad(int rank);

// Floats of split-K partial products launch_lora_xa_bf16 needs.
size_t lora_xa_partial_floats(int M, int K, int rank);

// xa[M, lora_pad(rank)] = scaling * (X A), zero past the rank, via
// part[lora_xa_partial_floats]; rank <= 64, K a multiple of 32.
hipError_t launch_lora_xa_bf16(const uint16_t* x, const float* a, int M, int K, int rank, float scaling, float* part,
                               float* xa, hipStream_t stream);

// Y[M, N] = X deq(W) (+ bias) (+ xa B); xa from launch_lora_xa_bf16 or null.
// The weight is in the reference's row-major layout, or striped
// (nf4_layout.hpp) when striped is set.
hipError_t launch_gemm(const uint16_t* x, const uint8_t* packed, const ScalesArg& scales, int M, int K, int N,
                       const float* bias, const float* lora_xa, const float* lora_b, int lora_rank, void* y,
                       bool y_bf16, bool striped, hipStream_t stream);

}  // namespace unifur
