// nf4_adapter_grad.hpp -- the LoRA adapter gradients of the QLoRA backward
// on f32 matrix cores (nf4_adapter_grad.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace unifur {

// True when the MFMA kernels take these operands: K and N multiples of 8
// (whole 8-element loads per lane), x, dy and B 16-byte aligned, rank in
// [1, 64], and rows of K or N values short enough for 32-bit buffer offsets
// over a workgroup's slab.  Otherwise the narrow VALU kernels of nf4_generic
// serve.
bool adapter_grads_supported(const void* x, const void* dy, const float* b, int M, int K, int N, int rank);

// Scratch for launch_adapter_grads: x A and dy B^T ([M][rank rounded up to
// 16, 32 or 64] f32 each) and the slab partials of the larger launch.
size_t adapter_grads_scratch_bytes(int M, int K, int N, int rank);

// grad_b [rank][N] = scaling (x A)^T dy and grad_a [K][rank] =
// scaling x^T (dy B^T) for x [M][K] and dy [M][N] (f32 or bf16), A [K][rank]
// and B [rank][N] (f32); either gradient may be null.  counters points at
// max_counters zeroed u32 that the launches leave zeroed (at most 512 are
// used).  M == 0 writes zero gradients.
hipError_t launch_adapter_grads(const void* x, bool x_bf16, const void* dy, bool dy_bf16, const float* a,
                                const float* b, int M, int K, int N, int rank, float scaling, float* grad_a,
                                float* grad_b, void* scratch, unsigned* counters, int max_counters,
                                hipStream_t stream);

// One row product on its own, out [M][adapter_row_product_ld(rank)] f32 at
// scratch (zero past the rank; slab partials after it): p = 0: x A with A
// [kdim][rank] (the forward adapter's first factor); p = 1: dy B^T with B
// [rank][kdim] (the backward dX adapter term's first factor).  src [M][kdim]
// f32 or bf16; the same operand conditions as the gradients (kdim % 8 == 0,
// src and w 16-byte aligned); counters as in launch_adapter_grads.
bool adapter_row_product_supported(const void* src, const float* w, int M, int kdim, int rank);
int adapter_row_product_ld(int rank);
size_t adapter_row_product_scratch_bytes(int M, int kdim, int rank);
hipError_t launch_adapter_row_product(int p, const void* src, bool src_bf16, const float* w, int M, int kdim,
                                      int rank, void* scratch, unsigned* counters, int max_counters,
                                      hipStream_t stream);

}  // namespace unifur
