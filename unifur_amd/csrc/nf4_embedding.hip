// nf4_embedding.hip -- Nf4Embedding::forward as a gather that dequantizes
// only the selected rows.
//
// The reference (src/qwennet.rs:244-291) holds a [n_embedding, d_model]
// table as one packed NF4 tensor with double quantization, dequantizes the
// whole table to f32 on every forward (5.1 GB for the 27B model) and then
// gathers rows with burn's embedding.  Here out[t][j] = the dequantized value
// of flat index ids[t] * d_model + j -- NF4_LEVELS[code] * block scale, the
// reference's f32 bit for bit (src/quantize.rs:355-366) -- for the gathered
// rows only: the bytes moved are the rows' codes and scales plus the output.
//
// When d_model % 8 == 0 each thread expands 8 consecutive values (one code
// dword, one block: 64 % 8 == 0) into two 16-byte f32 stores or one bf16
// store; otherwise one value per thread.  An id outside [0, n_embedding)
// yields a row of NaN (burn panics there; a kernel cannot, and a NaN row is
// what a consumer cannot mistake for data).
#include "nf4_embedding.hpp"

namespace unifur {
namespace {

template <typename Id>
__device__ __forceinline__ bool valid_id(Id id, uint64_t n) {
  return id >= 0 && (uint64_t)id < n;
}

__device__ __forceinline__ float block_scale(const ScalesArg& s, uint64_t b) {
  if (s.kind == kScalesDQ) return ((float)s.dq_codes[b] / 255.0f) * (*s.scale_of_scales);  // src/quantize.rs:349
  return s.absmax[b];
}

template <typename Id, bool BF16>
__global__ __launch_bounds__(256) void gather8_kernel(const uint8_t* __restrict__ packed, ScalesArg scales,
                                                      uint64_t n_embedding, uint64_t d_model,
                                                      const Id* __restrict__ ids, uint64_t n_ids, void* out) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) lut[threadIdx.x] = level((int)threadIdx.x);
  __syncthreads();
  const uint64_t per_row = d_model / 8;
  const uint64_t total = n_ids * per_row;
  for (uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
       g += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t t = g / per_row, q = g % per_row;
    const Id id = ids[t];
    float v[8];
    if (valid_id(id, n_embedding)) {
      const uint64_t i0 = (uint64_t)id * d_model + 8 * q;  // a multiple of 8: one code dword, one block
      const uint32_t code = *reinterpret_cast<const uint32_t*>(packed + i0 / 2);
      const float s = block_scale(scales, i0 / kBlock);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = lut[(code >> (4 * j)) & 15u] * s;  // NF4_LEVELS[c] * scale
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = __builtin_nanf("");
    }
    const uint64_t o = t * d_model + 8 * q;
    if constexpr (BF16) {
      const u32x4 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                       pack_bf16x2(v[6], v[7])};
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + o) = w;
    } else {
      f32x4* dst = reinterpret_cast<f32x4*>(static_cast<float*>(out) + o);
      dst[0] = f32x4{v[0], v[1], v[2], v[3]};
      dst[1] = f32x4{v[4], v[5], v[6], v[7]};
    }
  }
}

template <typename Id, bool BF16>
__global__ __launch_bounds__(256) void gather1_kernel(const uint8_t* __restrict__ packed, ScalesArg scales,
                                                      uint64_t n_embedding, uint64_t d_model,
                                                      const Id* __restrict__ ids, uint64_t n_ids, void* out) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) lut[threadIdx.x] = level((int)threadIdx.x);
  __syncthreads();
  const uint64_t total = n_ids * d_model;
  for (uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
       g += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t t = g / d_model, j = g % d_model;
    const Id id = ids[t];
    float v = __builtin_nanf("");
    if (valid_id(id, n_embedding)) {
      const uint64_t i = (uint64_t)id * d_model + j;
      const uint32_t c = (packed[i / 2] >> (4 * (i & 1))) & 15u;  // value 2m in the low nibble of byte m
      v = lut[c] * block_scale(scales, i / kBlock);
    }
    if constexpr (BF16)
      static_cast<uint16_t*>(out)[g] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
    else
      static_cast<float*>(out)[g] = v;
  }
}

template <typename Id, bool BF16>
hipError_t launch_typed(const uint8_t* packed, const ScalesArg& scales, uint64_t n_embedding, uint64_t d_model,
                        const Id* ids, uint64_t n_ids, void* out, bool vec, hipStream_t stream) {
  const uint64_t work = vec ? n_ids * (d_model / 8) : n_ids * d_model;
  const uint64_t blocks = (work + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
  if (vec)
    gather8_kernel<Id, BF16><<<grid, 256, 0, stream>>>(packed, scales, n_embedding, d_model, ids, n_ids, out);
  else
    gather1_kernel<Id, BF16><<<grid, 256, 0, stream>>>(packed, scales, n_embedding, d_model, ids, n_ids, out);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_embedding(const uint8_t* packed, const ScalesArg& scales, uint64_t n_embedding, uint64_t d_model,
                            const void* ids, bool ids_i64, uint64_t n_ids, void* out, bool bf16_out,
                            hipStream_t stream) {
  if (n_ids == 0 || d_model == 0) return hipSuccess;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(packed), oa = reinterpret_cast<uintptr_t>(out);
  const bool vec = d_model % 8 == 0 && (pa & 3u) == 0 && (oa & 15u) == 0;
  if (ids_i64) {
    const int64_t* p = static_cast<const int64_t*>(ids);
    return bf16_out ? launch_typed<int64_t, true>(packed, scales, n_embedding, d_model, p, n_ids, out, vec, stream)
                    : launch_typed<int64_t, false>(packed, scales, n_embedding, d_model, p, n_ids, out, vec, stream);
  }
  const int32_t* p = static_cast<const int32_t*>(ids);
  return bf16_out ? launch_typed<int32_t, true>(packed, scales, n_embedding, d_model, p, n_ids, out, vec, stream)
                  : launch_typed<int32_t, false>(packed, scales, n_embedding, d_model, p, n_ids, out, vec, stream);
}

}  // namespace unifur
