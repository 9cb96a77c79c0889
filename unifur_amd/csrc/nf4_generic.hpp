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
// y = x w^T with w stored [N, K] (same epilogue).
hipError_t launch_gemm_f32_wt(const void* x, bool x_bf16, const float* wt, int M, int K, int N, const Epilogue& e,
                              hipStream_t stream);
// xa[m][j] = sum_k x[m][k] a[k sk + j sj] (rank <= 64).
hipError_t launch_lora_xa_strided(const void* x, bool x_bf16, const float* a, size_t sk, size_t sj, int M, int K,
                                  int rank, float* xa, hipStream_t stream);
// c[P][Q] = scale * sum_m p[m][:]^T q[m][:] (p [M][P], q [M][Q]), summed over
// row slabs into partials (row_atb_slabs(M, P, Q) * P * Q floats) and then
// over the slabs in a fixed order.
int row_atb_slabs(int M, int P, int Q);
// out[m][j] = sum_k x[m][k] w(k, j) for j < rank <= 64, w(k, j) = w[k][j]
// (w [K][rank]) or, with w_t, w[j][k] (w [rank][K]); split over K into
// partials (narrow_mm_slabs(M, K) * M * rank floats), then summed in order.
int narrow_mm_slabs(int M, int K);
hipError_t launch_narrow_mm(const void* x, bool x_bf16, const float* w, bool w_t, int M, int K, int rank,
                            float* partials, float* out, hipStream_t stream);
// out = scale * sum_m wide[m][v] nar[m][j] (v < W, j < rank <= 64), stored
// [W][rank] or, with nar_major, [rank][W]; split over the rows into partials
// (narrow_atb_slabs(M, W) * W * rank floats), then summed in order.
int narrow_atb_slabs(int M, int W);
hipError_t launch_narrow_atb(const void* wide, bool wide_bf16, const float* nar, int M, int W, int rank,
                             bool nar_major, float scale, float* partials, float* out, hipStream_t stream);
hipError_t launch_row_atb(const void* p, bool p_bf16, const void* q, bool q_bf16, int M, int P, int Q, float scale,
                          float* partials, float* c, hipStream_t stream);
hipError_t launch_lora_merge(const float* w, const float* a, const float* b, int rank, float scaling, uint64_t K,
                             uint64_t N, float* out, hipStream_t stream);
hipError_t launch_silu_mul(const float* g, const float* u, size_t n, float* h, hipStream_t stream);
hipError_t launch_silu_mul_bf16(const float* g, const float* u, size_t n, uint16_t* h, hipStream_t stream);
// h[m][:] = bf16(silu(gu[m][:inter]) * gu[m][inter:]), gu [rows][2 inter] f32 or bf16.
hipError_t launch_silu_mul_rows_bf16(const void* gu, bool gu_f32, size_t rows, size_t inter, uint16_t* h,
                                     hipStream_t stream);
// QwenRmsNorm::forward (src/qwennet.rs:104-109) over the rows of x [rows, h]:
// out = (x * (mean(x^2) + eps)^(-1/2)) * (w + 1), f32 arithmetic, x and out
// f32 or bf16 (out rounded to nearest even).
hipError_t launch_rms_norm(const void* x, bool x_bf16, int rows, int h, const float* w, float eps, void* out,
                           bool out_bf16, hipStream_t stream);
// y = a + b elementwise over n values, each f32 or bf16 (the residual adds of
// QwenDecoderLayer::step, src/qwennet.rs:1124-1128).
hipError_t launch_add(const void* a, const void* b, bool bf16, size_t n, void* y, hipStream_t stream);

}  // namespace unifur
