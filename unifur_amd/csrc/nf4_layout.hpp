// nf4_layout.hpp -- the column-striped device layout of a linear weight.
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

// Columns per stripe: one stripe row is 8 bytes of packed codes.
constexpr int kStripeCols = 16;

// Codes of a [d_in, d_out] weight (d_out % 64 == 0, buffers 8-byte aligned)
// from the reference's row-major order to the striped order (to_striped) or
// back; src and dst are the buffers in the from and to orders.
hipError_t launch_stripe_codes(const uint8_t* src, uint8_t* dst, uint64_t d_in, uint64_t d_out, bool to_striped,
                               hipStream_t stream);

// Per-block scales (u8 DQ codes or f32 absmax) between [d_in, d_out / 64]
// (row-major) and [d_out / 64, d_in] (striped), the same way.
hipError_t launch_stripe_scales(const void* src, void* dst, uint64_t d_in, uint64_t d_out, bool dq, bool to_striped,
                                hipStream_t stream);

// dst [cols][rows] f32 = the transpose of src [rows][cols] (kSrcF32, or
// kSrcBf16 / kSrcF16 decoded exactly: nf4_common.hpp); rows up to 65535 * 64.
hipError_t launch_transpose_decode(const void* src, int src_kind, uint64_t rows, uint64_t cols, float* dst,
                                   hipStream_t stream);

}  // namespace unifur
