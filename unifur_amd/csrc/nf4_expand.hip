// nf4_expand.hip -- the NF4 weight expanded once per call to a bf16 operand
// for the prefill GEMM, with the LoRA update optionally merged into it.
//
// Wt[n][k] = bf16( L[c(k, n)] * scale(k, n / 64)  +  scaling * sum_r A[k][r] B[r][n] )
//
// W is the reference's packed [d_in = K, d_out = N] weight (src/qwennet.rs:
// 161-241): the first term is the reference's dequantized f32 value bit for
// bit (src/quantize.rs:355-366, level times block scale, one f32 multiply,
// DQ scale ((float)q / 255.0f) * sos); the second is the adapter's weight
// update (src/quantize.rs:619-624 computes (x A) B scaling, which equals
// x (A B scaling) up to rounding).  The sum is rounded to bf16 (RNE), the
// MFMA operand type.  Wt is stored output-column-major ([N][K], each
// column's K values contiguous): the "T" operand layout of a row-major
// Y = X Wt^T product, which the BLAS GEMM then streams with 16-byte loads.
//
// One 256-thread workgroup expands a 64 (k) x 64 (n) tile -- one NF4 block
// wide.  Thread t owns rows 2 (t % 32) and 2 (t % 32) + 1 and the 8 columns
// 8 (t / 32) .. + 7: one code dword per row, one scale per row.  The bf16
// (k, k + 1) pairs of each column go through an LDS transpose (row stride
// 36 dwords: the two column groups of a wave land on opposite bank halves)
// and leave as 128-byte column segments.  A workgroup takes up to four tiles
// along K, their loads all issued first.
#include "nf4_expand.hpp"

namespace unifur {
namespace {

constexpr int kTile = 64;
constexpr int kTStride = 36;                      // dwords per transposed column (32 + 4 pad)
constexpr int kLdsLut = 0;                        // NF4_LEVELS, 16 x f32
constexpr int kLdsT = 64;                         // KT transpose tiles of 64 x 36 dwords
constexpr int kTBytes = kTile * kTStride * 4;
constexpr int kMaxRank = 64;
constexpr int kCStride = 68;  // f32 per row of the LoRA product tile
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct ExpandArgs {
  const uint8_t* packed;
  ScalesArg scales;
  int K, N;
  const float* lora_a;  // [K][rank] or null
  const float* lora_b;  // [rank][N]
  int rank;
  float scaling;
  uint16_t* wt;  // [N][K]
  int tiles_k;   // K / 64
};

template <bool DQ, bool STRIPED, bool LORA, int KT>
__global__ __launch_bounds__(256) void expand_kernel(ExpandArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  // a workgroup expands KT tiles along K inside one 64-column band;
  // consecutive workgroups continue along K, so their output segments of each
  // column are adjacent
  const int groups_k = a.tiles_k / KT;
  const int k0 = (int)(blockIdx.x % (unsigned)groups_k) * (kTile * KT);
  const int n0 = (int)(blockIdx.x / (unsigned)groups_k) * kTile;
  const int kp = tid & 31, ng = tid >> 5;
  const int n = n0 + 8 * ng;

  // codes of rows k, k + 1 of every tile, columns n .. n + 7 (one dword
  // each), and the row scales of block n0 / 64: all loads first
  uint32_t code[KT][2];
  float s[KT][2];
  const int blk = n0 / kBlock;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const size_t row = (size_t)(k0 + kTile * t + 2 * kp + i);
      size_t sidx;
      if constexpr (STRIPED) {
        // stripe n / 16 holds 8 bytes per row; these 8 columns are its half (n % 16) / 8
        code[t][i] = *reinterpret_cast<const uint32_t*>(a.packed + ((size_t)(n / 16) * a.K + row) * 8 + (size_t)(ng & 1) * 4);
        sidx = (size_t)blk * a.K + row;
      } else {
        code[t][i] = *reinterpret_cast<const uint32_t*>(a.packed + row * (size_t)(a.N / 2) + n / 2);
        sidx = row * (size_t)(a.N / kBlock) + blk;
      }
      if constexpr (DQ)
        s[t][i] = ((float)a.scales.dq_codes[sidx] / 255.0f) * (*a.scales.scale_of_scales);  // src/quantize.rs:349
      else
        s[t][i] = a.scales.absmax[sidx];
    }

  float* lut = reinterpret_cast<float*>(smem + kLdsLut);
  if (tid < 16) lut[tid] = level(tid);
  // LoRA operands after the transpose tiles, bf16, zero past the rank (rank
  // rounded up to rp = 16, 32 or 64): A rows [64 KT][rp] and B transposed
  // [64 columns][rp], so that every MFMA fragment is one 16-byte read; then
  // the f32 product tile C [64][68]
  const int rp = a.rank <= 16 ? 16 : a.rank <= 32 ? 32 : 64;
  const int lds_a = kLdsT + KT * kTBytes, lds_b = lds_a + kTile * KT * rp * 2, lds_c = lds_b + kTile * rp * 2;
  if constexpr (LORA) {
    uint16_t* As = reinterpret_cast<uint16_t*>(smem + lds_a);
    uint16_t* Bt = reinterpret_cast<uint16_t*>(smem + lds_b);
    // A: four threads per row (columns tid % 4 + 4 j); B: one column per
    // thread (rows tid / 64 + 4 j)
    for (int kk = tid >> 2; kk < kTile * KT; kk += 64) {
      const float* arow = a.lora_a + (size_t)(k0 + kk) * a.rank;
      for (int r = tid & 3; r < rp; r += 4) As[kk * rp + r] = (uint16_t)pack_bf16x2(r < a.rank ? arow[r] : 0.0f, 0.0f);
    }
    const int nn = tid & 63;
    for (int r = tid >> 6; r < rp; r += 4)
      Bt[nn * rp + r] = (uint16_t)pack_bf16x2(r < a.rank ? a.lora_b[(size_t)r * a.N + n0 + nn] : 0.0f, 0.0f);
  }
  __syncthreads();

  uint32_t* T = reinterpret_cast<uint32_t*>(smem + kLdsT);
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    // v[i][j]: row k0 + 64 t + 2 kp + i, column n + j
    float v[2][8];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = lut[(code[t][i] >> (4 * j)) & 15u] * s[t][i];  // NF4_LEVELS[c] * scale
    if constexpr (LORA) {
      // C = A_t B for this tile: wave w computes the 32 x 32 block
      // (w / 2, w % 2) with rp / 16 v_mfma_f32_32x32x16_bf16 (bf16 factors,
      // f32 sums); C passes through LDS to the (k, k + 1) x 8-column layout
      const int lane = tid & 63, w = tid >> 6, bi = w >> 1, bj = w & 1, h = lane >> 5;
      const uint16_t* As = reinterpret_cast<const uint16_t*>(smem + lds_a);
      const uint16_t* Bt = reinterpret_cast<const uint16_t*>(smem + lds_b);
      float* C = reinterpret_cast<float*>(smem + lds_c);
      f32x16 acc = {};
      for (int r0 = 0; r0 < rp; r0 += 16) {
        const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(As + (kTile * t + 32 * bi + (lane & 31)) * rp + r0 + 8 * h);
        const bf16x8_t bf = *reinterpret_cast<const bf16x8_t*>(Bt + (32 * bj + (lane & 31)) * rp + r0 + 8 * h);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc, 0, 0, 0);
      }
      if (t > 0) __syncthreads();  // the previous tile's C has been read
      // acc[4 q + e] = C[8 q + 4 h + e][lane % 32] of the block
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) C[(32 * bi + 8 * q + 4 * h + e) * kCStride + 32 * bj + (lane & 31)] = acc[4 * q + e];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f32x4* cr = reinterpret_cast<const f32x4*>(C + (2 * kp + i) * kCStride + 8 * ng);
        const f32x4 c0 = cr[0], c1 = cr[1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[i][j] += a.scaling * c0[j];
          v[i][j + 4] += a.scaling * c1[j];
        }
      }
    }
    // transpose through tile buffer t: column 8 ng + j, dword kp = bf16 pair (k, k + 1)
    uint32_t* Tt = T + t * (kTile * kTStride);
#pragma unroll
    for (int j = 0; j < 8; ++j) Tt[(8 * ng + j) * kTStride + kp] = pack_bf16x2(v[0][j], v[1][j]);
  }
  __syncthreads();
  // column c = t / 4, quarter q = t % 4: 16 k values of each tile = two
  // 16-byte stores per tile
  const int c = tid >> 2, q = tid & 3;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const u32x4* src = reinterpret_cast<const u32x4*>(T + t * (kTile * kTStride) + c * kTStride + 8 * q);
    u32x4* dst = reinterpret_cast<u32x4*>(a.wt + (size_t)(n0 + c) * a.K + k0 + kTile * t + 16 * q);
    dst[0] = src[0];
    dst[1] = src[1];
  }
}

// LDS of a KT-tile workgroup: the transpose tiles, then with an adapter its
// bf16 A rows and B columns and the f32 product tile.
size_t expand_smem(int KT, int rank) {
  const size_t rp = rank <= 16 ? 16 : rank <= 32 ? 32 : 64;
  return kLdsT + (size_t)KT * kTBytes + (rank ? (size_t)kTile * KT * rp * 2 + kTile * rp * 2 + kTile * kCStride * 4 : 0);
}

template <bool DQ, bool STRIPED, bool LORA>
hipError_t launch_t(const ExpandArgs& a, hipStream_t stream) {
  const long long band = a.N / kTile;
  // without an adapter four (or two) tiles per workgroup where K allows:
  // more loads in flight; with one, one tile (its LDS would otherwise limit
  // the workgroups per CU, which measured slower)
  if constexpr (!LORA) {
    if (a.tiles_k % 4 == 0) {
      expand_kernel<DQ, STRIPED, false, 4><<<(int)(band * (a.tiles_k / 4)), 256, expand_smem(4, 0), stream>>>(a);
      return hipGetLastError();
    }
    if (a.tiles_k % 2 == 0) {
      expand_kernel<DQ, STRIPED, false, 2><<<(int)(band * (a.tiles_k / 2)), 256, expand_smem(2, 0), stream>>>(a);
      return hipGetLastError();
    }
  }
  expand_kernel<DQ, STRIPED, LORA, 1><<<(int)(band * a.tiles_k), 256, expand_smem(1, a.rank), stream>>>(a);
  return hipGetLastError();
}

}  // namespace

bool expand_supported(int K, int N, int rank) {
  return K > 0 && N > 0 && K % kTile == 0 && N % kTile == 0 && rank >= 0 && rank <= kMaxRank;
}

hipError_t launch_expand_bf16(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                              const float* lora_a, const float* lora_b, int rank, float scaling, uint16_t* wt,
                              hipStream_t stream) {
  if (!expand_supported(K, N, rank) || (rank > 0 && (!lora_a || !lora_b))) return hipErrorInvalidValue;
  ExpandArgs a{};
  a.packed = packed;
  a.scales = scales;
  a.K = K;
  a.N = N;
  a.lora_a = lora_a;
  a.lora_b = lora_b;
  a.rank = rank;
  a.scaling = scaling;
  a.wt = wt;
  a.tiles_k = K / kTile;
  const long long tiles = (long long)(K / kTile) * (N / kTile);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const bool dq = scales.kind == kScalesDQ;
  const bool lora = rank > 0;
  if (dq) {
    if (striped) return lora ? launch_t<true, true, true>(a, stream) : launch_t<true, true, false>(a, stream);
    return lora ? launch_t<true, false, true>(a, stream) : launch_t<true, false, false>(a, stream);
  }
  if (striped) return lora ? launch_t<false, true, true>(a, stream) : launch_t<false, true, false>(a, stream);
  return lora ? launch_t<false, false, true>(a, stream) : launch_t<false, false, false>(a, stream);
}

}  // namespace unifur
