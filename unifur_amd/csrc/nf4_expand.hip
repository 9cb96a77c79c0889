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

#include <algorithm>

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
  const float* la;  // A f32 [K][rank]
  const float* lb;  // B f32 [rank][N]
  int la_vec;       // rank % 8 == 0 and A 16-byte aligned: fragments of A in two 16-byte loads
  int rank, rp;
  float scaling;
  uint16_t* wt;  // [N][K]
  int tiles_k;   // K / 64
  int n_base;    // first column of the launch (a multiple of 64)
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
  const int n0 = a.n_base + (int)(blockIdx.x / (unsigned)groups_k) * kTile;
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
  // LoRA: the MFMA fragments straight from the f32 factors, issued with the
  // code loads and rounded to bf16 in registers (A: eight consecutive values
  // of a row; B^T: eight rows of a column, coalesced across the lanes); the
  // f32 product tile C [64][68] after the transpose tiles
  const int lane = tid & 63, wv = tid >> 6, bi = wv >> 1, bj = wv & 1, h = lane >> 5;
  const int lds_c = kLdsT + KT * kTBytes;
  // adapter fragments per tile: up to rank 64 in the one-tile kernel, rank
  // 16 (one fragment) when a workgroup takes several tiles
  constexpr int kMaxFr = (LORA && KT == 1) ? kMaxRank / 16 : 1;
  bf16x8_t bfr[kMaxFr];
  bf16x8_t afr[KT][kMaxFr];
  if constexpr (LORA) {
    const int nf = a.rp / 16;
#pragma unroll
    for (int f = 0; f < kMaxFr; ++f) {
      if (f >= nf) break;
      const int r0 = 16 * f + 8 * h;  // this lane's eight adapter indices
      const size_t col = (size_t)(n0 + 32 * bj + (lane & 31));
      float bv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = r0 + e < a.rank ? a.lb[(size_t)(r0 + e) * a.N + col] : 0.0f;
      bfr[f] = __builtin_bit_cast(bf16x8_t, u32x4{pack_bf16x2(bv[0], bv[1]), pack_bf16x2(bv[2], bv[3]),
                                                  pack_bf16x2(bv[4], bv[5]), pack_bf16x2(bv[6], bv[7])});
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const size_t row = (size_t)(k0 + kTile * t + 32 * bi + (lane & 31));
        float av[8];
        if (a.la_vec) {
          f32x4 lo = {0.0f, 0.0f, 0.0f, 0.0f}, hi = lo;
          if (r0 < a.rank) {
            const f32x4* src = reinterpret_cast<const f32x4*>(a.la + row * a.rank + r0);
            lo = src[0];
            hi = src[1];
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            av[e] = lo[e];
            av[4 + e] = hi[e];
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) av[e] = r0 + e < a.rank ? a.la[row * a.rank + r0 + e] : 0.0f;
        }
        afr[t][f] = __builtin_bit_cast(bf16x8_t, u32x4{pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3]),
                                                       pack_bf16x2(av[4], av[5]), pack_bf16x2(av[6], av[7])});
      }
    }
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
      float* C = reinterpret_cast<float*>(smem + lds_c);
      f32x16 acc = {};
#pragma unroll
      for (int f = 0; f < kMaxFr; ++f) {
        if (f >= a.rp / 16) break;
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[t][f], bfr[f], acc, 0, 0, 0);
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

// LDS of a KT-tile workgroup: the transpose tiles, then with an adapter the
// f32 product tile.
size_t expand_smem(int KT, bool lora) {
  return kLdsT + (size_t)KT * kTBytes + (lora ? (size_t)kTile * kCStride * 4 : 0);
}

template <bool DQ, bool STRIPED, bool LORA>
hipError_t launch_t(const ExpandArgs& a, int n_count, hipStream_t stream) {
  const long long band = n_count / kTile;
  // four (or two) tiles per workgroup where K allows: more loads in flight
  // (with an adapter of rank <= 16, whose fragments then fit the registers)
  if (LORA && a.rp > 16) {
    expand_kernel<DQ, STRIPED, LORA, 1><<<(int)(band * a.tiles_k), 256, expand_smem(1, LORA), stream>>>(a);
    return hipGetLastError();
  }
  if (a.tiles_k % 4 == 0) {
    expand_kernel<DQ, STRIPED, LORA, 4><<<(int)(band * (a.tiles_k / 4)), 256, expand_smem(4, LORA), stream>>>(a);
    return hipGetLastError();
  }
  if (a.tiles_k % 2 == 0) {
    expand_kernel<DQ, STRIPED, LORA, 2><<<(int)(band * (a.tiles_k / 2)), 256, expand_smem(2, LORA), stream>>>(a);
    return hipGetLastError();
  }
  expand_kernel<DQ, STRIPED, LORA, 1><<<(int)(band * a.tiles_k), 256, expand_smem(1, LORA), stream>>>(a);
  return hipGetLastError();
}

}  // namespace

bool expand_supported(int K, int N, int rank) {
  return K > 0 && N > 0 && K % kTile == 0 && N % kTile == 0 && rank >= 0 && rank <= kMaxRank;
}


hipError_t launch_expand_bf16(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                              const float* lora_a, const float* lora_b, int rank, float scaling, uint16_t* wt,
                              hipStream_t stream) {
  return launch_expand_cols(packed, scales, K, N, striped, lora_a, lora_b, rank, scaling, 0, N, wt, stream);
}

hipError_t launch_expand_cols(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                              const float* lora_a, const float* lora_b, int rank, float scaling, int n_begin, int n_end,
                              uint16_t* wt, hipStream_t stream) {
  if (!expand_supported(K, N, rank) || (rank > 0 && (!lora_a || !lora_b)) || n_begin < 0 || n_end > N ||
      n_begin % kTile != 0 || n_end % kTile != 0 || n_begin >= n_end)
    return hipErrorInvalidValue;
  const int rp = rank <= 16 ? 16 : rank <= 32 ? 32 : 64;
  ExpandArgs a{};
  a.packed = packed;
  a.scales = scales;
  a.K = K;
  a.N = N;
  a.la = lora_a;
  a.lb = lora_b;
  a.la_vec = rank % 8 == 0 && (reinterpret_cast<uintptr_t>(lora_a) & 15u) == 0;
  a.rank = rank;
  a.rp = rp;
  a.scaling = scaling;
  a.wt = wt;
  a.tiles_k = K / kTile;
  a.n_base = n_begin;
  const int nc = n_end - n_begin;
  const long long tiles = (long long)(K / kTile) * (nc / kTile);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const bool dq = scales.kind == kScalesDQ;
  const bool lora = rank > 0;
  if (dq) {
    if (striped) return lora ? launch_t<true, true, true>(a, nc, stream) : launch_t<true, true, false>(a, nc, stream);
    return lora ? launch_t<true, false, true>(a, nc, stream) : launch_t<true, false, false>(a, nc, stream);
  }
  if (striped) return lora ? launch_t<false, true, true>(a, nc, stream) : launch_t<false, true, false>(a, nc, stream);
  return lora ? launch_t<false, false, true>(a, nc, stream) : launch_t<false, false, false>(a, nc, stream);
}

}  // namespace unifur
