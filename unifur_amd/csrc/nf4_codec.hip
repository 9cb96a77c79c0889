// nf4_codec.hip -- blockwise absmax NF4 quantize / double-quantize / dequantize.
//
// Bit-exact restatement of src/quantize.rs:99-124 (quantize), :129-149 and
// :284-309 (double quantization), :169-185 and :329-366 (dequantize) as
// gfx950 kernels.  Every f32 operation that the reference performs is
// performed here with the same operands in the same order (IEEE RN, no
// contraction), so codes, bytes, absmax, DQ codes and dequantized f32 values
// equal the reference's.
#include "nf4_codec.hpp"

#pragma clang fp contract(off)

namespace unifur {
namespace {

// Half-width of the window around a threshold where the quantizer's fast
// reciprocal path defers to the exact division: 2^-20 >= 4x the 2^-22 by
// which v * rcp(absmax) can differ from fl(v / absmax) for |u| <= 1.
constexpr float kNear = 9.5367431640625e-07f;

// Exact decision thresholds of nearest_level_code (src/quantize.rs:208-219):
// for u in [-1, 1], scan(u) == #{t : u >= T[t]}.  Each T[t] is the smallest
// f32 at which the strict-< scan over f32 distances first returns code t+1;
// nine of them sit one ulp away from the f32 midpoint of adjacent levels.
__constant__ uint32_t kThresholdBits[15] = {
    0xbf591cd8u, 0xbf1c5270u, 0xbeeb847fu, 0xbeadea76u, 0xbe703cecu,
    0xbe0d38bbu, 0xbd3a7870u, 0x3d22fb00u, 0x3df64863u, 0x3e5067e1u,
    0x3e9582d5u, 0x3ec753fau, 0x3f006d04u, 0x3f248db0u, 0x3f5c89dau};

// Bucket table over floor(16 u) in [-16, 16]: no two thresholds are closer
// than 1/16, so bucket j holds at most one threshold.  Entry j stores
// {count of thresholds <= j/16, the threshold inside the bucket or 2.0f}.
struct BucketEntry {
  float t_in;
  uint32_t base;
};

__device__ __forceinline__ void build_bucket_table(BucketEntry* tab) {
  for (int j = threadIdx.x; j < 33; j += blockDim.x) {
    float lo = (float)(j - 16) * 0.0625f;
    float hi = lo + 0.0625f;
    uint32_t base = 0;
    float t_in = 2.0f;
    for (int t = 0; t < 15; ++t) {
      float T = __uint_as_float(kThresholdBits[t]);
      if (T <= lo) base++;
      else if (T < hi) t_in = T;
    }
    tab[j] = BucketEntry{t_in, base};
  }
}

// scan(u) for u = v / absmax in [-1, 1] or NaN.  u * 16 is exact (power of
// two).  fmaxf/fminf are IEEE maxNum/minNum, so a NaN u clamps to bucket 0,
// whose base is 0 and whose compare is false: NaN -> code 0, as the scan.
__device__ __forceinline__ uint32_t code_of(float u, const BucketEntry* tab) {
  float s = fminf(fmaxf(__builtin_floorf(u * 16.0f), -16.0f), 16.0f);
  BucketEntry e = tab[(int)s + 16];
  return e.base + (u >= e.t_in ? 1u : 0u);
}

// ---------------------------------------------------------------- quantize --
// One wave covers 16 blocks (1024 values, 4 KiB) per step.  Load instruction
// q of lane l reads float4 #(q*64 + l) of the wave's span, so every load is a
// contiguous 1 KiB across the wave and block (q*4 + l/16) lives in the 16
// consecutive lanes of one instruction: absmax is a 16-lane max reduction.
//
// The code of v is scan(fl(v / absmax)).  The IEEE division costs a dozen
// instructions, so the kernel first classifies u' = v * rcp(absmax), which
// is within 3 ulp of fl(v / absmax) whenever absmax is a normal f32 (rcp is
// 1 ulp, the product 1/2 ulp).  scan is a step function whose steps sit at
// the 15 thresholds, none of them within 2^-9 of a bucket edge, so u' and
// fl(v / absmax) get the same code unless u' lies within kNear of the
// threshold inside its bucket; those values, and every value of a block
// whose absmax is zero, subnormal or not finite, take the exact division.
constexpr int kQuantWaves = 4;  // waves per workgroup
constexpr int kQuantThreads = kQuantWaves * 64;

// Max over the 16 lanes of each row, in every lane: DPP quad_perm [1,0,3,2]
// and [2,3,0,1], then row_half_mirror and row_mirror (every lane of a quad,
// then of a half row, then of the row holds the max of the span so far).
// NaN never reaches here (inputs pass through fabs + fmax with 0 start), so
// the order of the butterfly does not matter.
// The values are >= 0 and never NaN, so their bit patterns order like the
// values and the steps are integer maxes (no canonicalisation).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return dpp_mov<CTRL>(v);
}
__device__ __forceinline__ float max16(float f) {
  uint32_t v = __float_as_uint(f);
  v = max(v, dpp_u<0xB1>(v));
  v = max(v, dpp_u<0x4E>(v));
  v = max(v, dpp_u<0x141>(v));
  v = max(v, dpp_u<0x140>(v));
  return __uint_as_float(v);
}

// Code of v from u = v * rcp(absmax); `near` is set when u lies within kNear
// of the threshold of its bucket (the caller then divides exactly).
__device__ __forceinline__ uint32_t code_fast(float v, float r, const BucketEntry* tab, bool& near) {
  const float u = v * r;
  // bucket floor(16 u) + 16, by truncation of 16 u + 16 >= 0 (u >= -1 - 3 ulp;
  // a bucket off by one next to an edge gives the same code, see above);
  // a NaN u takes bucket 0: code 0, as the scan
  const float t = __builtin_fmaf(u, 16.0f, 16.0f);
  const uint32_t b = (uint32_t)fminf(fmaxf(t, 0.0f), 32.0f);  // < 0 and NaN -> 0 (maxNum)
  const BucketEntry e = tab[b];
  near = near || fabsf(u - e.t_in) <= kNear;
  return e.base + (u >= e.t_in ? 1u : 0u);
}

__device__ __forceinline__ uint32_t code_exact(float v, float m, const BucketEntry* tab) {
  return m == 0.0f ? 7u : code_of(v / m, tab);
}

__global__ __launch_bounds__(kQuantThreads) void quantize_full_kernel(
    const float* __restrict__ values, uint8_t* __restrict__ packed, float* __restrict__ absmax,
    size_t n_full_spans) {
  __shared__ BucketEntry tab[33];
  build_bucket_table(tab);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const size_t wave = (size_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  const size_t nwaves = (size_t)gridDim.x * kQuantWaves;
  for (size_t span = wave; span < n_full_spans; span += nwaves) {
    const f32x4* src = reinterpret_cast<const f32x4*>(values) + span * 256;
    f32x4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = __builtin_nontemporal_load(src + q * 64 + lane);
    float m[4];
    uint32_t nib[4];
    bool exact = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // absmax = fold(0, max(acc, |v|)) (src/quantize.rs:103); fmaxf is
      // IEEE maxNum, so NaN inputs are ignored exactly as Rust's f32::max.
      m[q] = fmaxf(fmaxf(fmaxf(0.0f, fabsf(v[q].x)), fmaxf(fabsf(v[q].y), fabsf(v[q].z))), fabsf(v[q].w));
      m[q] = max16(m[q]);
      // rcp(m) is a normal f32 for m in [2^-126, 2^126]; outside (m == 0:
      // all codes 7, src/quantize.rs:108-110) the block takes the exact path
      exact = exact || !(m[q] >= 1.1754943508222875e-38f && m[q] <= 8.507059173023462e+37f);
      const float r = __builtin_amdgcn_rcpf(m[q]);
      nib[q] = code_fast(v[q].x, r, tab, exact) | (code_fast(v[q].y, r, tab, exact) << 4) |
               (code_fast(v[q].z, r, tab, exact) << 8) | (code_fast(v[q].w, r, tab, exact) << 12);
    }
    if (exact) {  // rare: this lane's 16 values by the exact division
#pragma unroll
      for (int q = 0; q < 4; ++q)
        nib[q] = code_exact(v[q].x, m[q], tab) | (code_exact(v[q].y, m[q], tab) << 4) |
                 (code_exact(v[q].z, m[q], tab) << 8) | (code_exact(v[q].w, m[q], tab) << 12);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const size_t f4 = span * 256 + q * 64 + lane;  // float4 index == u16 index of packed
      reinterpret_cast<uint16_t*>(packed)[f4] = (uint16_t)nib[q];
      if ((lane & 15) == 0) absmax[f4 / 16] = m[q];
    }
  }
}

// Tail (fewer than 1024 values): one thread per block, scalar, any n.
__global__ void quantize_tail_kernel(const float* __restrict__ values, uint8_t* __restrict__ packed,
                                     float* __restrict__ absmax, size_t first_block, size_t n) {
  __shared__ BucketEntry tab[33];
  build_bucket_table(tab);
  __syncthreads();
  size_t b = first_block + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t start = b * kBlock;
  if (start >= n) return;
  size_t end = start + kBlock < n ? start + kBlock : n;
  float m = 0.0f;
  for (size_t i = start; i < end; ++i) m = fmaxf(m, fabsf(values[i]));
  for (size_t i = start; i < end; i += 2) {
    uint32_t lo = m == 0.0f ? 7u : code_of(values[i] / m, tab);
    uint32_t hi = 0;
    if (i + 1 < end) hi = m == 0.0f ? 7u : code_of(values[i + 1] / m, tab);
    packed[i / 2] = (uint8_t)(lo | (hi << 4));
  }
  absmax[b] = m;
}

// ------------------------------------------------------- double quantize --
// Pass 1: max over the f32 absmax values.  All are >= 0 and never NaN (they
// come out of a NaN-ignoring max from 0), so their bit patterns order like
// the values and an integer atomic max is exact.  Pass 2 encodes.
// The global max of the block scales: a grid-stride max per thread, the
// workgroup's max through LDS, then one atomic max per workgroup.  The grid
// is capped at kDqMaxBlocks: the atomics on the one address serialise (one
// per wave over a 1024-workgroup grid took config 1's 262,144 scales 48 us).
constexpr int kDqMaxBlocks = 64;
__global__ __launch_bounds__(256) void dq_max_kernel(const float* __restrict__ absmax, size_t nb,
                                                     uint32_t* __restrict__ max_bits) {
  __shared__ float wave_max[4];
  float m = 0.0f;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nb; i += (size_t)gridDim.x * blockDim.x)
    m = fmaxf(m, absmax[i]);
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  m = fmaxf(m, __shfl_xor(m, 4));
  m = fmaxf(m, __shfl_xor(m, 8));
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
    atomicMax(max_bits, __float_as_uint(m));
  }
}

__global__ void zero_u32_kernel(uint32_t* p) { *p = 0u; }

__global__ void dq_encode_kernel(const float* __restrict__ absmax, size_t nb, const uint32_t* __restrict__ max_bits,
                                 uint8_t* __restrict__ q) {
  const float M = __uint_as_float(*max_bits);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nb; i += (size_t)gridDim.x * blockDim.x) {
    uint8_t c = 0;
    if (M != 0.0f) {
      // (s / max_scale * 255.0).round().clamp(0.0, 255.0) as u8
      float r = roundf((absmax[i] / M) * 255.0f);  // half away from zero
      c = (r == r) ? (uint8_t)fminf(fmaxf(r, 0.0f), 255.0f) : (uint8_t)0;
    }
    q[i] = c;
  }
}

// -------------------------------------------------------------- dequantize --
// LUT in LDS: byte b -> {level[b & 15], level[b >> 4]}, kDeqLutCopies copies
// (lane l reads copy l % kDeqLutCopies: the random 8-byte reads of a wave
// spread over the banks).  The DQ scale is ((float)q / 255.0f) * sos,
// evaluated as the reference does, once per code in an LDS table.
constexpr int kDeqLutCopies = 8;

// NF4_LEVELS[c] for a per-lane c from immediates (no memory access)
__device__ __forceinline__ float level_of(int c) {
  float v = level(0);
#pragma unroll
  for (int i = 1; i < 16; ++i) v = c == i ? level(i) : v;
  return v;
}

__device__ __forceinline__ float block_scale(const ScalesArg& s, size_t blk) {
  if (s.kind == kScalesF32) return s.absmax[blk];
  return ((float)s.dq_codes[blk] / 255.0f) * (*s.scale_of_scales);
}

// A wave covers kDeqTiles tiles of 512 values (128 float4) per step: lane l
// expands the four values of float4 l and of float4 64 + l of each tile (two
// code bytes each), so each store is a contiguous 1 KiB across the wave and
// each code load a contiguous 128 bytes; 16 lanes share a 64-value block.
// All loads of a step are issued before its lookups and stores.
constexpr int kDeqTiles = 8;

template <bool kBf16Out, bool kDQ>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ packed, ScalesArg scales,
                                                         size_t n_tiles, void* __restrict__ out) {
  __shared__ f32x2 lut[256 * kDeqLutCopies];
  __shared__ float dq_lut[256];
  {
    const int b = threadIdx.x;  // 256 threads: entry b, all its copies
    const f32x2 e = {level_of(b & 15), level_of(b >> 4)};
#pragma unroll
    for (int c = 0; c < kDeqLutCopies; ++c) lut[b * kDeqLutCopies + c] = e;
    if constexpr (kDQ) dq_lut[b] = ((float)b / 255.0f) * (*scales.scale_of_scales);  // src/quantize.rs:349
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int copy = lane % kDeqLutCopies;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(packed);
  const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const size_t nwaves = (size_t)gridDim.x * 4;
  for (size_t t0 = wave * kDeqTiles; t0 < n_tiles; t0 += nwaves * kDeqTiles) {
    uint32_t w[kDeqTiles][2], sc[kDeqTiles][2];  // code bytes; scale (f32 bits or DQ code)
#pragma unroll
    for (int u = 0; u < kDeqTiles; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const size_t f4 = (t0 + u) * 128 + h * 64 + lane;  // float4 index == u16 index of the codes
        const bool ok = t0 + u < n_tiles;
        w[u][h] = ok ? __builtin_nontemporal_load(src + f4) : 0u;
        if constexpr (kDQ)
          sc[u][h] = ok ? scales.dq_codes[f4 / 16] : 0u;
        else
          sc[u][h] = ok ? __float_as_uint(scales.absmax[f4 / 16]) : 0u;
      }
#pragma unroll
    for (int u = 0; u < kDeqTiles; ++u) {
      if (t0 + u >= n_tiles) break;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const size_t f4 = (t0 + u) * 128 + h * 64 + lane;
        const float s = kDQ ? dq_lut[sc[u][h]] : __uint_as_float(sc[u][h]);
        const f32x2 p0 = lut[(w[u][h] & 0xff) * kDeqLutCopies + copy], p1 = lut[(w[u][h] >> 8) * kDeqLutCopies + copy];
        // out = NF4_LEVELS[c] * scale: one f32 multiply, as src/quantize.rs:362
        const float o0 = p0.x * s, o1 = p0.y * s, o2 = p1.x * s, o3 = p1.y * s;
        if constexpr (kBf16Out) {
          const u32x2 r = {pack_bf16x2(o0, o1), pack_bf16x2(o2, o3)};
          __builtin_nontemporal_store(r, reinterpret_cast<u32x2*>(out) + f4);
        } else {
          __builtin_nontemporal_store(f32x4{o0, o1, o2, o3}, reinterpret_cast<f32x4*>(out) + f4);
        }
      }
    }
  }
}

// Tail: values [first, n), one thread per value.
template <bool kBf16Out>
__global__ void dequantize_tail_kernel(const uint8_t* __restrict__ packed, ScalesArg scales, size_t first, size_t n,
                                       void* __restrict__ out) {
  size_t i = first + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint8_t byte = packed[i / 2];
  uint32_t c = (i & 1) ? (byte >> 4) : (byte & 15);
  float o = level(c) * block_scale(scales, i / kBlock);
  if constexpr (kBf16Out) {
    reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)(pack_bf16x2(o, 0.0f) & 0xffffu);
  } else {
    reinterpret_cast<float*>(out)[i] = o;
  }
}

// ------------------------------------------------------ transpose-quantize --
// The loader's step (src/qwennet.rs:1687-1726): a checkpoint weight
// src[out_f][in_f] (PyTorch [out, in], f32, or bf16 / f16 decoded exactly as
// src/import.rs:255-272 does) is transposed to [in_f][out_f] (transpose2d,
// src/qwennet.rs:1375-1390) and quantized (PackedNf4Tensor::quantize) -- here
// in one pass, without the transposed f32 copy.  With out_f % 64 == 0 every
// 64-value block of the transposed buffer is 64 consecutive output features
// of one input feature, i.e. one column segment of a 64 x 64 source tile.
// Tile in LDS (padded rows), then wave lane l takes block row k = l / 4 of
// its 16 and the quarter l % 4 of the block: a 4-lane absmax, 16 codes, one
// 8-byte store.  Arithmetic identical to quantize_full_kernel.
template <int SRC>
__global__ __launch_bounds__(256) void quantize_transposed_kernel(const void* __restrict__ src, uint64_t out_f,
                                                                  uint64_t in_f, uint8_t* __restrict__ packed,
                                                                  float* __restrict__ absmax) {
  __shared__ BucketEntry tab[33];
  __shared__ float tile[64][65];
  build_bucket_table(tab);
  const int tid = threadIdx.x;
  const uint64_t o0 = (uint64_t)blockIdx.y * 64, k0 = (uint64_t)blockIdx.x * 64;
  // load: tile[o][k] = src[o0 + o][k0 + k], rows of 64 consecutive values
  for (int i = tid; i < 64 * 64; i += 256) {
    const int o = i >> 6, k = i & 63;
    float v = 0.0f;
    if (k0 + k < in_f) {
      const uint64_t idx = (o0 + o) * in_f + k0 + k;
      v = decode_src<SRC>(src, idx);
    }
    tile[o][k] = v;
  }
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  const int q = lane & 3;              // quarter of the 64-value block
  const int kr = wave * 16 + (lane >> 2);  // tile row k: four waves x 16 rows
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = tile[q * 16 + i][kr];
  // absmax = fold(0, max(acc, |v|)) over the block (src/quantize.rs:103),
  // NaN-ignoring maxNum as Rust's f32::max
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
  m = fmaxf(m, __shfl_xor(m, 1, 4));
  m = fmaxf(m, __shfl_xor(m, 2, 4));
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t c = m == 0.0f ? 7u : code_of(v[i] / m, tab);  // src/quantize.rs:104-114
    if (i < 8)
      lo |= c << (4 * i);
    else
      hi |= c << (4 * (i - 8));
  }
  if (k0 + kr < in_f) {
    const uint64_t base = (k0 + kr) * out_f + o0 + (uint64_t)q * 16;  // value index in [in_f][out_f]
    reinterpret_cast<uint2*>(packed)[base / 16] = make_uint2(lo, hi);
    if (q == 0) absmax[base / 64] = m;
  }
}

int grid_for(size_t work_items, int threads, int max_blocks) {
  size_t g = (work_items + threads - 1) / threads;
  if (g > (size_t)max_blocks) g = max_blocks;
  return g < 1 ? 1 : (int)g;
}

// ------------------------------------------------- grouped linear quantize --
// The quantize pass of a model's linears in three launches per group of up
// to kQGroupMax tensors instead of ~6 per tensor: each tensor is a
// row-major f32 [K, N] weight (N % 64 == 0) quantized with double
// quantization straight into the striped resident form.  The arithmetic is
// quantize_full_kernel's and dq_encode_kernel's, so codes, DQ codes and the
// scale of scales equal quantize + double quantize + stripe of the tensor.
//   1. a wave per span of 16 rows x one 64-column block: codes of block
//      (k, b) go to the stripes 4b .. 4b+3 at row k -- 8 bytes each, stripe s
//      holding K rows of 8 bytes, so a span writes 128 contiguous bytes per
//      stripe -- and its f32 absmax to absmax_tmp[b K + k], the striped
//      scale order
//   2. the max of each tensor's block scales (one workgroup per tensor; an
//      atomic max per wave instead serialises on one address per tensor)
//   3. encode absmax_tmp against the max into the u8 scales, same order
constexpr int kQGroupMax = 48;

struct QGroupTensor {
  const float* values;  // [K][N] f32, 16-byte aligned
  uint8_t* packed;      // striped codes, K N / 2 bytes, 8-byte aligned
  uint8_t* dq;          // u8 scales [N / 64][K]
  float* absmax;        // workspace f32 [N / 64][K]
  uint32_t* max_bits;   // the scale of scales (device f32), written as its bits
  uint32_t K, N;
  uint32_t span_begin;  // first span of this tensor in the group
};

struct QGroupArgs {
  int n;
  uint32_t spans;  // over the group
  QGroupTensor t[kQGroupMax];
};

// Which tensor of the group holds a span, by one ballot: lane i < n holds
// tensor i's fields (loaded once per wave), the span's tensor is the last
// whose first span it reaches, and its fields come back by readlane -- a few
// scalar instructions per span instead of a chain of dependent scalar loads
// from the kernel arguments (a binary search over them cost a grouped pass
// over config 5's weights 300 us against 215 us for the same reads alone).
struct LaneTensor {
  uint64_t values, packed, absmax;
  uint32_t K, N, begin;
};
struct SpanTensor {
  const void* values;
  uint8_t* packed;
  float* absmax;
  uint32_t K, N, local;  // local: the span's index inside its tensor
};
static_assert(kQGroupMax <= 64, "one lane per tensor of a group");

__device__ __forceinline__ LaneTensor lane_tensor(const QGroupArgs& a, int lane) {
  LaneTensor t{0, 0, 0, 0, 0, 0xffffffffu};
  if (lane < a.n) {
    const QGroupTensor& T = a.t[lane];
    t = LaneTensor{(uint64_t)(uintptr_t)T.values, (uint64_t)(uintptr_t)T.packed, (uint64_t)(uintptr_t)T.absmax,
                   T.K, T.N, T.span_begin};
  }
  return t;
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ SpanTensor span_tensor(const LaneTensor& t, uint32_t span) {
  const int i = __popcll(__ballot(span >= t.begin)) - 1;  // tensor 0 begins at span 0
  SpanTensor s;
  s.values = reinterpret_cast<const void*>(readlane64(t.values, i));
  s.packed = reinterpret_cast<uint8_t*>(readlane64(t.packed, i));
  s.absmax = reinterpret_cast<float*>(readlane64(t.absmax, i));
  s.K = __builtin_amdgcn_readlane(t.K, i);
  s.N = __builtin_amdgcn_readlane(t.N, i);
  s.local = span - __builtin_amdgcn_readlane(t.begin, i);
  return s;
}

__global__ __launch_bounds__(kQuantThreads) void qgroup_quantize_kernel(QGroupArgs a) {
  __shared__ BucketEntry tab[33];
  // per wave: the span's codes as [stripe][row][u16 part] and its 16 scales
  __shared__ __attribute__((aligned(16))) uint16_t stage[kQuantWaves][4 * 16 * 4];
  __shared__ float stage_m[kQuantWaves][16];
  build_bucket_table(tab);
  __syncthreads();
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const LaneTensor lt = lane_tensor(a, lane);
  const uint32_t nwaves = gridDim.x * kQuantWaves;
  for (uint32_t span = blockIdx.x * kQuantWaves + wv; span < a.spans; span += nwaves) {
    const SpanTensor T = span_tensor(lt, span);
    // span = (16-row group rg, block column b): block q * 4 + lane / 16 of
    // the wave is row 16 rg + 4 q + lane / 16, columns 64 b .. 64 b + 63, so
    // each stripe of the block gets 16 consecutive rows = 128 contiguous
    // bytes from this wave, and the block scales 16 consecutive entries
    const uint32_t bpr = T.N / kBlock;
    const uint32_t rg = T.local / bpr, b = T.local - rg * bpr;
    const uint32_t c = lane & 15;  // values 4c .. 4c + 3 of the block: columns 64 b + 4 c ..
    const float* values = static_cast<const float*>(T.values);
    f32x4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t k = 16 * rg + 4 * q + lane / 16;
      v[q] = k < T.K ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(values + (size_t)k * T.N + 64 * b) + c)
                     : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    float m[4];
    uint32_t nib[4];
    bool exact = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // absmax = fold(0, max(acc, |v|)) (src/quantize.rs:103), as quantize_full_kernel
      m[q] = fmaxf(fmaxf(fmaxf(0.0f, fabsf(v[q].x)), fmaxf(fabsf(v[q].y), fabsf(v[q].z))), fabsf(v[q].w));
      m[q] = max16(m[q]);
      exact = exact || !(m[q] >= 1.1754943508222875e-38f && m[q] <= 8.507059173023462e+37f);
      const float r = __builtin_amdgcn_rcpf(m[q]);
      nib[q] = code_fast(v[q].x, r, tab, exact) | (code_fast(v[q].y, r, tab, exact) << 4) |
               (code_fast(v[q].z, r, tab, exact) << 8) | (code_fast(v[q].w, r, tab, exact) << 12);
    }
    if (exact) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        nib[q] = code_exact(v[q].x, m[q], tab) | (code_exact(v[q].y, m[q], tab) << 4) |
                 (code_exact(v[q].z, m[q], tab) << 8) | (code_exact(v[q].w, m[q], tab) << 12);
    }
    // Through the wave's LDS slot, so that each lane stores one row's 8
    // bytes of one stripe (lane l: stripe 4 b + l / 16, row 16 rg + l % 16)
    // instead of four 2-byte pieces: scattered 2-byte stores cost the pass
    // more than its arithmetic.  One wave writes and reads its own slot; the
    // wave barriers keep the compiler from moving the accesses across.
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      stage[wv][((c / 4) * 16 + 4 * q + lane / 16) * 4 + (c & 3)] = (uint16_t)nib[q];
      if (c == 0) stage_m[wv][4 * q + lane / 16] = m[q];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t k = 16 * rg + (lane & 15);
    if (k < T.K) {
      const uint64_t stripe = 4ull * b + (uint32_t)lane / 16;
      *reinterpret_cast<u32x2*>(T.packed + (stripe * T.K + k) * 8) =
          *reinterpret_cast<const u32x2*>(&stage[wv][lane * 4]);
      if (lane < 16) T.absmax[(uint64_t)b * T.K + k] = stage_m[wv][lane];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
}

// The same first pass from checkpoint tensors as they lie: values[i] is the
// PyTorch-order [N][K] weight (f32, or bf16 / f16 decoded exactly), i.e. the
// transpose of the [K][N] weight to quantize (qwen_linear's transpose2d,
// src/qwennet.rs:1375-1390, fused away).  A workgroup per 64 x 64 source
// tile (k tile kt, block column b): rows o = 64 b .. + 63 of the source,
// columns k = 64 kt .. + 63, through LDS (padded rows); then wave w takes
// tile rows k = 16 w .. + 15, lane l block row k = 16 w + l / 4 and the
// quarter q = l % 4 of its 64 values, which is exactly stripe 4 b + q of
// that row: a 4-lane absmax, 16 codes, one 8-byte store (the four lanes of
// a row write its four stripes, the 16 rows of a wave 128 contiguous bytes
// per stripe).  VEC: rows 16-byte aligned (K a multiple of 8 for bf16 and
// f16, 4 for f32), the tile loaded 16 bytes per thread and load.
template <int SRC, bool VEC>
__global__ __launch_bounds__(256) void qgroup_quantize_t_kernel(QGroupArgs a) {
  constexpr bool HALF = SRC != kSrcF32;  // 2-byte elements
  __shared__ BucketEntry tab[33];
  __shared__ float tile[64][65];
  build_bucket_table(tab);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const LaneTensor lt = lane_tensor(a, lane);
  for (uint32_t span = blockIdx.x; span < a.spans; span += gridDim.x) {
    const SpanTensor T = span_tensor(lt, span);  // the tensor holding this tile (each wave alike)
    const uint32_t bpr = T.N / kBlock;
    const uint32_t kt = T.local / bpr, b = T.local - kt * bpr;
    const uint32_t k0 = 64u * kt;
    const uint64_t o0 = 64ull * b;
    __syncthreads();  // the bucket table built; the previous tile's reads done
    if constexpr (VEC) {
      constexpr int kPer = HALF ? 8 : 4;  // values per 16-byte load
      constexpr int kRowLoads = 64 / kPer;
      for (int i = tid; i < 64 * kRowLoads; i += 256) {
        const int o = i / kRowLoads, kc = (i % kRowLoads) * kPer;
        float v[kPer];
        if (k0 + kc < T.K) {  // K is a multiple of kPer: the load lies inside the row
          const uint64_t idx = (o0 + o) * T.K + k0 + kc;
          const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(T.values) +
                                                          idx * (HALF ? 2 : 4));
          if constexpr (HALF) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[2 * e] = decode_half<SRC>(w[e] & 0xffffu);
              v[2 * e + 1] = decode_half<SRC>(w[e] >> 16);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(w[e]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < kPer; ++e) v[e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < kPer; ++e) tile[o][kc + e] = v[e];
      }
    } else {
      for (int i = tid; i < 64 * 64; i += 256) {
        const int o = i >> 6, k = i & 63;
        float v = 0.0f;
        if (k0 + k < T.K) {
          const uint64_t idx = (o0 + o) * T.K + k0 + k;
          v = decode_src<SRC>(T.values, idx);
        }
        tile[o][k] = v;
      }
    }
    __syncthreads();
    const int q = lane & 3;
    const int kr = wave * 16 + (lane >> 2);
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = tile[q * 16 + i][kr];
    // absmax = fold(0, max(acc, |v|)) over the block (src/quantize.rs:103)
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1, 4));
    m = fmaxf(m, __shfl_xor(m, 2, 4));
    // the codes as quantize_full_kernel: classify v * rcp(absmax), divide
    // exactly near a threshold or for an absmax outside the normal range
    bool exact = !(m >= 1.1754943508222875e-38f && m <= 8.507059173023462e+37f);
    const float r = __builtin_amdgcn_rcpf(m);
    uint32_t c[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) c[i] = code_fast(v[i], r, tab, exact);
    if (exact) {
#pragma unroll
      for (int i = 0; i < 16; ++i) c[i] = code_exact(v[i], m, tab);
    }
    uint32_t w0 = 0, w1 = 0;  // byte j: codes of columns 2 j (low nibble) and 2 j + 1
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w0 |= c[i] << (4 * i);
      w1 |= c[8 + i] << (4 * i);
    }
    const uint32_t k = k0 + (uint32_t)kr;
    if (k < T.K) {
      const uint64_t stripe = 4ull * b + (uint64_t)q;
      *reinterpret_cast<u32x2*>(T.packed + (stripe * T.K + k) * 8) = u32x2{w0, w1};
      if (q == 0) T.absmax[(uint64_t)b * T.K + k] = m;
    }
  }
}

// The scale of scales of tensor blockIdx.x: the max of its block scales
// (src/quantize.rs:285-290), one workgroup per tensor.  The values are >= 0
// and never NaN, so the order of the max does not matter.
__global__ __launch_bounds__(1024) void qgroup_max_kernel(QGroupArgs a) {
  __shared__ float wm[16];
  const QGroupTensor& T = a.t[blockIdx.x];
  const uint64_t nb = (uint64_t)T.K * (T.N / kBlock);
  float m = 0.0f;
  const uint64_t step = blockDim.x;
  for (uint64_t i0 = threadIdx.x; i0 < nb; i0 += 8 * step) {  // eight loads in flight per thread
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = i0 + u * step < nb ? T.absmax[i0 + u * step] : 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) m = fmaxf(m, v[u]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, wm[w]);
    *T.max_bits = __float_as_uint(r);
  }
}

__global__ void qgroup_encode_kernel(QGroupArgs a) {
  const QGroupTensor& T = a.t[blockIdx.y];
  const float M = __uint_as_float(*T.max_bits);
  const uint64_t nb = (uint64_t)T.K * (T.N / kBlock);
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nb; i += (uint64_t)gridDim.x * blockDim.x) {
    uint8_t c = 0;
    if (M != 0.0f) {
      // (s / max_scale * 255.0).round().clamp(0.0, 255.0) as u8 (src/quantize.rs:285-303)
      const float r = roundf((T.absmax[i] / M) * 255.0f);  // half away from zero
      c = (r == r) ? (uint8_t)fminf(fmaxf(r, 0.0f), 255.0f) : (uint8_t)0;
    }
    T.dq[i] = c;
  }
}

}  // namespace

hipError_t launch_quantize(const float* values, size_t n, uint8_t* packed, float* absmax, bool aligned,
                           hipStream_t stream) {
  if (n == 0) return hipSuccess;
  // full 16-block spans take the vector kernel (needs 16-byte aligned values
  // and 2-byte aligned codes); the rest, or everything if misaligned, the
  // scalar one.
  const size_t spans = aligned ? n / 1024 : 0;
  if (spans) {
    int grid = grid_for(spans, kQuantWaves, 8192);
    quantize_full_kernel<<<grid, kQuantThreads, 0, stream>>>(values, packed, absmax, spans);
  }
  const size_t first_block = spans * 16;
  const size_t nb = (n + kBlock - 1) / kBlock;
  if (first_block < nb) {
    size_t tail_blocks = nb - first_block;
    quantize_tail_kernel<<<(unsigned)((tail_blocks + 63) / 64), 64, 0, stream>>>(values, packed, absmax,
                                                                              first_block, n);
  }
  return hipGetLastError();
}

hipError_t launch_double_quantize(const float* absmax, size_t nb, uint8_t* q, float* scale_of_scales,
                                  hipStream_t stream) {
  // The scale of scales is the max itself, so its own storage is the
  // accumulator of the integer atomic max (non-negative f32 bits order as u32).
  // (zeroed by a kernel rather than a memset node, so that the call can be
  // captured in a graph)
  uint32_t* max_bits = reinterpret_cast<uint32_t*>(scale_of_scales);
  zero_u32_kernel<<<1, 1, 0, stream>>>(max_bits);
  if (nb == 0) return hipGetLastError();
  dq_max_kernel<<<grid_for(nb, 256, kDqMaxBlocks), 256, 0, stream>>>(absmax, nb, max_bits);
  dq_encode_kernel<<<grid_for(nb, 256, 4096), 256, 0, stream>>>(absmax, nb, max_bits, q);
  return hipGetLastError();
}

hipError_t launch_dequantize(const uint8_t* packed, const ScalesArg& scales, size_t n, void* out, bool bf16_out,
                             bool aligned, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  // tiles of 512 values take the vector kernel (2-byte aligned codes,
  // 16-byte aligned output); the remainder, or everything if misaligned, the
  // scalar one.
  const size_t tiles = aligned ? n / 512 : 0;
  if (tiles) {
    const int grid = grid_for(tiles, 4 * kDeqTiles, 8192);
    const bool dq = scales.kind == kScalesDQ;
    if (bf16_out)
      dq ? dequantize_kernel<true, true><<<grid, 256, 0, stream>>>(packed, scales, tiles, out)
         : dequantize_kernel<true, false><<<grid, 256, 0, stream>>>(packed, scales, tiles, out);
    else
      dq ? dequantize_kernel<false, true><<<grid, 256, 0, stream>>>(packed, scales, tiles, out)
         : dequantize_kernel<false, false><<<grid, 256, 0, stream>>>(packed, scales, tiles, out);
  }
  const size_t first = tiles * 512;
  if (first < n) {
    unsigned g = (unsigned)((n - first + 63) / 64);
    if (bf16_out)
      dequantize_tail_kernel<true><<<g, 64, 0, stream>>>(packed, scales, first, n, out);
    else
      dequantize_tail_kernel<false><<<g, 64, 0, stream>>>(packed, scales, first, n, out);
  }
  return hipGetLastError();
}

hipError_t launch_quantize_transposed(const void* src, int src_kind, uint64_t out_f, uint64_t in_f, uint8_t* packed,
                                      float* absmax, hipStream_t stream) {
  if (out_f == 0 || in_f == 0) return hipSuccess;
  const uint64_t gx = (in_f + 63) / 64, gy = out_f / 64;
  if (out_f % 64 != 0 || gx > 0x7fffffffu || gy > 65535u) return hipErrorInvalidValue;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  switch (src_kind) {
    case kSrcF32: quantize_transposed_kernel<kSrcF32><<<grid, 256, 0, stream>>>(src, out_f, in_f, packed, absmax); break;
    case kSrcBf16: quantize_transposed_kernel<kSrcBf16><<<grid, 256, 0, stream>>>(src, out_f, in_f, packed, absmax); break;
    case kSrcF16: quantize_transposed_kernel<kSrcF16><<<grid, 256, 0, stream>>>(src, out_f, in_f, packed, absmax); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}


// The simulated form's storage (src/quantize.rs:68-95): one code per byte.
// Thread i owns packed byte i, i.e. values 2i and 2i + 1 (low nibble first,
// src/quantize.rs:329-337).  Unpack writes both codes (only the first when
// 2i + 1 is past the end); pack joins them, with a zero high nibble for an
// odd length's last byte, as PackedNf4Tensor::quantize does
// (src/quantize.rs:266-273).
__global__ __launch_bounds__(256) void unpack_codes_kernel(const uint8_t* __restrict__ packed, size_t len,
                                                           uint8_t* __restrict__ codes) {
  const size_t bytes = (len + 1) / 2;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes; i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t b = packed[i];
    codes[2 * i] = (uint8_t)(b & 15u);
    if (2 * i + 1 < len) codes[2 * i + 1] = (uint8_t)(b >> 4);
  }
}

__global__ __launch_bounds__(256) void pack_codes_kernel(const uint8_t* __restrict__ codes, size_t len,
                                                         uint8_t* __restrict__ packed) {
  const size_t bytes = (len + 1) / 2;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes; i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t lo = codes[2 * i] & 15u;
    const uint32_t hi = 2 * i + 1 < len ? (codes[2 * i + 1] & 15u) : 0u;
    packed[i] = (uint8_t)(lo | (hi << 4));
  }
}

hipError_t launch_unpack_codes(const uint8_t* packed, size_t len, uint8_t* codes, hipStream_t stream) {
  if (len == 0) return hipSuccess;
  unpack_codes_kernel<<<grid_for((len + 1) / 2, 256, 8192), 256, 0, stream>>>(packed, len, codes);
  return hipGetLastError();
}

hipError_t launch_pack_codes(const uint8_t* codes, size_t len, uint8_t* packed, hipStream_t stream) {
  if (len == 0) return hipSuccess;
  pack_codes_kernel<<<grid_for((len + 1) / 2, 256, 8192), 256, 0, stream>>>(codes, len, packed);
  return hipGetLastError();
}

size_t quantize_linears_scratch_bytes(const uint64_t* d_in, const uint64_t* d_out, uint32_t n) {
  size_t total = 0;
  for (uint32_t i = 0; i < n; ++i) total += ((size_t)(d_in[i] * (d_out[i] / kBlock) * 4) + 255) & ~size_t{255};
  return total;
}

hipError_t launch_quantize_linears(const void* const* values, int src_kind, const uint64_t* d_in,
                                   const uint64_t* d_out, uint32_t n, uint8_t* const* packed, uint8_t* const* dq,
                                   float* const* sos, void* scratch, hipStream_t stream) {
  const bool transposed = src_kind != kQuantSrcF32;
  const bool half = src_kind == kQuantSrcBf16T || src_kind == kQuantSrcF16T;
  char* tmp = static_cast<char*>(scratch);
  for (uint32_t g0 = 0; g0 < n; g0 += kQGroupMax) {
    QGroupArgs a{};
    a.n = (int)std::min<uint32_t>(kQGroupMax, n - g0);
    uint64_t spans = 0, max_nb = 0;
    bool vec = true;
    for (int i = 0; i < a.n; ++i) {
      const uint32_t j = g0 + i;
      QGroupTensor& T = a.t[i];
      T.values = static_cast<const float*>(values[j]);
      T.packed = packed[j];
      T.dq = dq[j];
      T.absmax = reinterpret_cast<float*>(tmp);
      T.max_bits = reinterpret_cast<uint32_t*>(sos[j]);
      T.K = (uint32_t)d_in[j];
      T.N = (uint32_t)d_out[j];
      T.span_begin = (uint32_t)spans;
      const uint64_t nb = d_in[j] * (d_out[j] / kBlock);
      tmp += ((size_t)nb * 4 + 255) & ~size_t{255};
      // 16-row groups (64-row source tiles when transposed) x block columns
      spans += (d_in[j] + (transposed ? 63 : 15)) / (transposed ? 64 : 16) * (d_out[j] / kBlock);
      max_nb = std::max(max_nb, nb);
      vec = vec && (reinterpret_cast<uintptr_t>(values[j]) & 15u) == 0 && d_in[j] % (half ? 8 : 4) == 0;
    }
    if (spans > 0xffffffffull) return hipErrorInvalidValue;
    a.spans = (uint32_t)spans;
    if (spans && !transposed) {
      qgroup_quantize_kernel<<<grid_for(spans, kQuantWaves, 8192), kQuantThreads, 0, stream>>>(a);
    } else if (spans) {
      const int grid = (int)std::min<uint64_t>(spans, 8192);
      if (src_kind == kQuantSrcBf16T)
        vec ? qgroup_quantize_t_kernel<kSrcBf16, true><<<grid, 256, 0, stream>>>(a)
            : qgroup_quantize_t_kernel<kSrcBf16, false><<<grid, 256, 0, stream>>>(a);
      else if (src_kind == kQuantSrcF16T)
        vec ? qgroup_quantize_t_kernel<kSrcF16, true><<<grid, 256, 0, stream>>>(a)
            : qgroup_quantize_t_kernel<kSrcF16, false><<<grid, 256, 0, stream>>>(a);
      else
        vec ? qgroup_quantize_t_kernel<kSrcF32, true><<<grid, 256, 0, stream>>>(a)
            : qgroup_quantize_t_kernel<kSrcF32, false><<<grid, 256, 0, stream>>>(a);
    }
    qgroup_max_kernel<<<(unsigned)a.n, 1024, 0, stream>>>(a);
    if (max_nb) {
      const unsigned gx = (unsigned)std::min<uint64_t>((max_nb + 255) / 256, 256);
      qgroup_encode_kernel<<<dim3(gx, (unsigned)a.n), 256, 0, stream>>>(a);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace unifur
