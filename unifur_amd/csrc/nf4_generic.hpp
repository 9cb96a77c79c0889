// nf4_generic.hpp -- internal interface of the shape-general linear pieces.
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

// Output stage shared by the linear kernels: y = acc (+ bias) (+ LoRA).
struct Epilogue {
  const float* bias;     // [N] or null
  const float* lora_xa;  // [M, lora_rank] = x A, or null
  const float* lora_b;   // [lora_rank, N]
  int lora_rank;
  float lora_scaling;
  void* y;  // [M, N] f32 or bf16
  int y_bf16;
};

hipError_t launch_gemm_f32(const void* x, bool x_bf16, const float* w, int M, int K, int N, const Epilogue& e,
                           hipStream_t stream);
hipError_t launch_lora_xa(const void* x, bool x_bf16, const float* a, int M, int K, int rank, float* xa,
                          hipStream_t stream);
hipError_t launch_lora_merge(const float* w, const float* a, const float* b, int rank, float scaling, uint64_t K,
                             uint64_t N, float* out, hipStream_t stream);
hipError_t launch_silu_mul(const float* g, const float* u, size_t n, float* h, hipStream_t stream);
hipError_t launch_silu_mul_bf16(const float* g, const float* u, size_t n, uint16_t* h, hipStream_t stream);

}  // namespace unifur
