// nf4_embedding.hpp -- gather-dequantize of an NF4 embedding table.
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

// out[t][:] = dequantized row ids[t] of the [n_embedding, d_model] table
// (f32 bit-exact, or bf16 = RNE of it); rows of NaN for ids out of range.
hipError_t launch_embedding(const uint8_t* packed, const ScalesArg& scales, uint64_t n_embedding, uint64_t d_model,
                            const void* ids, bool ids_i64, uint64_t n_ids, void* out, bool bf16_out,
                            hipStream_t stream);

}  // namespace unifur
