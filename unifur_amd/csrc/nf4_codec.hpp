// nf4_codec.hpp -- internal launcher declarations shared by the C-ABI layer.
#pragma once

#include "nf4_common.hpp"

namespace unifur {

enum : int { kScalesF32 = 0, kScalesDQ = 1 };

// Per-block scales as the kernels receive them (device pointers).
struct ScalesArg {
  int kind;                      // kScalesF32 or kScalesDQ
  const float* absmax;           // kScalesF32: one f32 per block
  const uint8_t* dq_codes;       // kScalesDQ: one u8 per block
  const float* scale_of_scales;  // kScalesDQ: one f32 (device)
};

hipError_t launch_quantize(const float* values, size_t n, uint8_t* packed, float* absmax, bool aligned,
                           hipStream_t stream);
hipError_t launch_double_quantize(const float* absmax, size_t nb, uint8_t* q, float* scale_of_scales,
                                  hipStream_t stream);
// src[out_f][in_f] (kSrcF32, kSrcBf16 or kSrcF16: nf4_common.hpp) -> packed
// NF4 codes and f32 absmax of its [in_f][out_f] transpose; out_f % 64 == 0,
// packed 8-byte aligned.
hipError_t launch_quantize_transposed(const void* src, int src_kind, uint64_t out_f, uint64_t in_f, uint8_t* packed,
                                      float* absmax, hipStream_t stream);
hipError_t launch_dequantize(const uint8_t* packed, const ScalesArg& scales, size_t n, void* out, bool bf16_out,
                             bool aligned, hipStream_t stream);
// One code per byte (the simulated Nf4Tensor's storage) <-> two per byte.
hipError_t launch_unpack_codes(const uint8_t* packed, size_t len, uint8_t* codes, hipStream_t stream);
hipError_t launch_pack_codes(const uint8_t* codes, size_t len, uint8_t* packed, hipStream_t stream);
// The quantize pass of n linears: row-major f32 values[i] [d_in[i], d_out[i]]
// (d_out % 64 == 0, values 16-byte and packed 8-byte aligned) quantized with
// double quantization into the striped resident form (packed[i] striped
// codes, dq[i] u8 scales [d_out / 64][d_in], sos[i] the scale of scales),
// three launches per group of up to 48 tensors; scratch holds the f32 block
// scales (quantize_linears_scratch_bytes).
size_t quantize_linears_scratch_bytes(const uint64_t* d_in, const uint64_t* d_out, uint32_t n);
// src_kind: kQuantSrcF32 -- values[i] f32 [d_in][d_out] (16-byte
// aligned); kQuantSrcF32T / kQuantSrcBf16T / kQuantSrcF16T -- the
// PyTorch-order [d_out][d_in] tensor (f32, or bf16 / f16 decoded exactly),
// transposed on the fly, 4- or 2-byte aligned.  The outputs are the same for a tensor and its
// transposed copy.
enum { kQuantSrcF32 = 0, kQuantSrcF32T = 1, kQuantSrcBf16T = 2, kQuantSrcF16T = 3 };
hipError_t launch_quantize_linears(const void* const* values, int src_kind, const uint64_t* d_in,
                                   const uint64_t* d_out, uint32_t n, uint8_t* const* packed, uint8_t* const* dq,
                                   float* const* sos, void* scratch, hipStream_t stream);

}  // namespace unifur
