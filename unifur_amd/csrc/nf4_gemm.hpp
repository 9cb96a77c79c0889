// nf4_gemm.hpp -- internal interface of the MFMA prefill GEMM.
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

// Shapes and buffers the MFMA GEMM takes: bf16 X 16-byte aligned, K a
// multiple of 64, N a multiple of 128 (whole 128 x 128 tiles along N; rows
// past M are masked), (M + 256) K bf16 values under 2 GiB (32-bit buffer
// offsets).
bool gemm_supported(int M, int K, int N, const void* x);

// Adapter columns padded to a multiple of 16 (the row stride of the LoRA
// operand buffers below).
int lora_pad(int rank);

// The fused LoRA epilogue's operands, bf16: at[pad][K] (A transposed, a
// scratch operand), bt[N][pad] (B transposed) and xa[M][pad] =
// scaling * (X A), zero past the rank; rank <= 64, K a multiple of 64.
hipError_t launch_lora_operands(const uint16_t* x, const float* a, const float* b, int M, int K, int N, int rank,
                                float scaling, uint16_t* at, uint16_t* bt, uint16_t* xa, hipStream_t stream);

// Y[M, N] = X deq(W) (+ bias) (+ xa B); xa and bt from launch_lora_operands, or null.
// The weight is in the reference's row-major layout, or striped
// (nf4_layout.hpp) when striped is set.
// With k_splits > 1 (no adapter, y 16-byte aligned) the workgroups of a
// tile split d_in and write f32 sums to partials (k_splits * M * N floats),
// which a second launch adds in split order with the bias and rounding.
hipError_t launch_gemm(const uint16_t* x, const uint8_t* packed, const ScalesArg& scales, int M, int K, int N,
                       const float* bias, const uint16_t* lora_xa, const uint16_t* lora_bt, int lora_rank, void* y,
                       bool y_bf16, bool striped, hipStream_t stream, int k_splits = 1, float* partials = nullptr,
                       int tail_splits = 1);

// SwiGLU gate/up pair: h[M, N] = bf16(silu(X deq(gate)) * (X deq(up))),
// both weights [K, N] of one layout and scale kind, N a multiple of 64, h
// 8-byte aligned for its fast stores.  One launch: a workgroup computes 64
// columns of both weights over 256 rows and forms the product in
// registers.  With k_splits > 1 the workgroups of a tile split d_in and
// write raw f32 sums to partials (k_splits * M * 2 N floats), which a second
// launch adds in split order before the product.
hipError_t launch_gemm_pair(const uint16_t* x, const uint8_t* gate_packed, const ScalesArg& gate_scales,
                            const uint8_t* up_packed, const ScalesArg& up_scales, int M, int K, int N, uint16_t* h,
                            bool striped, hipStream_t stream, int k_splits = 1, float* partials = nullptr,
                            int tail_splits = 1);

// dX[M, d_in] = dY[M, d_out] deq(W)^T (+ lora_xa lora_bt^T) for a striped
// weight W [d_in, d_out] (d_in a multiple of 128): the fused kernel with the
// weight's rows as its outputs, each W tile dequantized once per 256 rows of
// dY.  The adapter operands come from launch_lora_operands_dx; k_splits as
// in launch_gemm (split over d_out, no adapter).
hipError_t launch_gemm_dx(const uint16_t* dy, const uint8_t* packed, const ScalesArg& scales, int M, int d_in, int d_out,
                          const uint16_t* lora_xa, const uint16_t* lora_bt, int lora_rank, void* dx, bool dx_bf16,
                          hipStream_t stream, int k_splits = 1, float* partials = nullptr);

// The adapter operands of dX's epilogue: dX gains ((dY scaling) B^T) A^T,
// so at = B [pad][d_out] and bt = A [d_in][pad] in bf16, and xa =
// bf16(scaling dY B^T) [M][pad]; d_out a multiple of 64.
hipError_t launch_lora_operands_dx(const uint16_t* dy, const float* a, const float* b, int M, int d_in, int d_out,
                                   int rank, float scaling, uint16_t* at, uint16_t* bt, uint16_t* xa,
                                   hipStream_t stream);

// tail_splits > 1 (k_splits 1, no adapter, y 16-byte aligned; partials as
// for k_splits = tail_splits): the tiles of the grid's whole rounds run
// whole and those of its last, partly filled round split d_in
// tail_splits ways, with an ordered reduction of just those tiles.
// gemm_tail_splits gives the count for a shape (1: no tail split).
int gemm_tail_splits(int M, int K, int N, bool pair = false);

// d_in slabs the fused GEMM splits into for this shape (1: no split); pair:
// the gate/up pair launch over two [K, N] weights.
int gemm_k_splits(int M, int K, int N, bool pair = false);

}  // namespace unifur
