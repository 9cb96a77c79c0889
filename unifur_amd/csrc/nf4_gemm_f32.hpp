// nf4_gemm_f32.hpp -- internal interface of the f32 MFMA GEMM over an NF4
// weight (f32 activations or f32 dY at batch sizes past the skinny kernel).
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

struct F32GemmArgs {
  const float* x;  // [M][K] f32, 16-byte aligned (K the reduction dim)
  const uint8_t* packed;  // the stored weight [d_in][d_out], row-major or striped
  ScalesArg scales;
  int M, K, N;  // rows, reduction, outputs: (M, d_in, d_out), or with trans (M, d_out, d_in)
  const float* bias;      // [N] or null
  const float* lora_xa;   // [M][lora_ld] f32 (x A, or dY B^T with trans; lora_rank columns used), or null
  int lora_ld;
  const float* lora_b;    // element (j, n) of the second factor at lora_b[j lora_sbj + n lora_sbn]
  size_t lora_sbj, lora_sbn;
  int lora_rank;
  float lora_scaling;
  void* y;  // [M][N] f32 or bf16
};

// Shapes the kernel takes: M, Kr, N > 0, the reduction dim Kr a multiple of
// 4, the stored weight's d_out a multiple of 64, x 16-byte aligned.
bool gemm_f32_mfma_supported(int M, int Kr, int N, int w_d_out, const void* x);

// y = x deq(W) (+ bias) (+ scaling xa B) -- or with trans y = x deq(W)^T
// (+ scaling xa B'), B' read through the strides -- in f32 on MFMA, the
// weight operand level * scale exactly (the reference's dequantized f32).
hipError_t launch_gemm_f32_mfma(const F32GemmArgs& g, bool dq, bool striped, bool trans, bool y_bf16,
                                hipStream_t stream);

}  // namespace unifur
