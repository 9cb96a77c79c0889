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
// wide -- or up to four of them along K, their loads all issued first.
// Without an adapter thread t owns rows 2 (t % 32) and 2 (t % 32) + 1 and
// the 8 columns 8 (t / 32) .. + 7: one code dword per row, one scale per
// row, and each column's bf16 (k, k + 1) pair is one dword of Wt; for one
// column the 32 lanes of a half-wave write 32 consecutive pairs, a 128-byte
// segment, so the output needs no LDS transpose.
#include "nf4_expand.hpp"

#include <algorithm>

namespace unifur {
namespace {

constexpr int kTile = 64;
constexpr int kLdsLut = 0;                        // NF4_LEVELS, 16 x f32 per wave
constexpr int kLdsBytes = 256;                        // LDS bytes: the four waves' LUTs
constexpr int kMaxRank = 64;
constexpr int kRowPitch = 144;                    // LDS bytes per row of a ROWS tile (64 bf16 + 16: two-way banks)
constexpr int kRowTileBytes = 64 * kRowPitch;
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct ExpandArgs {
  const uint8_t* packed;
  ScalesArg scales;
  int K, N;
  const float* la;  // A f32 [K][rank]
  const float* lb;  // B f32 [rank][N]
  int la_vec;       // rank % 8 == 0 and A 16-byte aligned: fragments of A in two 16-byte loads
  int stage;        // rank 16, A and B 16-byte aligned: fragments staged through LDS
  int rank, rp;
  float scaling;
  uint16_t* wt;  // [N][K]
  int tiles_k;   // K / 64
  int n_base;    // first column of the launch (a multiple of 64)
};

// Codes of rows k, k + 1 of a 64 x 64 tile for columns n .. n + 7 and the
// rows' scales of block n0 / 64.
template <bool DQ, bool STRIPED>
__device__ __forceinline__ void load_row_codes(const ExpandArgs& a, size_t row, int n, int ng, int blk, uint32_t& code,
                                               float& s) {
  size_t sidx;
  if constexpr (STRIPED) {
    // stripe n / 16 holds 8 bytes per row; these 8 columns are its half (n % 16) / 8
    code = *reinterpret_cast<const uint32_t*>(a.packed + ((size_t)(n / 16) * a.K + row) * 8 + (size_t)(ng & 1) * 4);
    sidx = (size_t)blk * a.K + row;
  } else {
    code = *reinterpret_cast<const uint32_t*>(a.packed + row * (size_t)(a.N / 2) + n / 2);
    sidx = row * (size_t)(a.N / kBlock) + blk;
  }
  if constexpr (DQ)
    s = ((float)a.scales.dq_codes[sidx] / 255.0f) * (*a.scales.scale_of_scales);  // src/quantize.rs:349
  else
    s = a.scales.absmax[sidx];
}

template <bool DQ, bool STRIPED, int KT>
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
    for (int i = 0; i < 2; ++i)
      load_row_codes<DQ, STRIPED>(a, (size_t)(k0 + kTile * t + 2 * kp + i), n, ng, blk, code[t][i], s[t][i]);

  // one LUT copy per wave: no workgroup barrier
  const int lane = tid & 63, wv = tid >> 6;
  float* lut = reinterpret_cast<float*>(smem + kLdsLut) + 16 * wv;
  if (lane < 16) lut[lane] = level(lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // the bf16 (k, k + 1) pair of column n + j goes straight to Wt: for one
  // j the 32 lanes of a half-wave write 32 consecutive pairs of that
  // column, one 128-byte segment
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(a.wt + (size_t)n * a.K + k0 + kTile * t) + kp;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v0 = lut[(code[t][0] >> (4 * j)) & 15u] * s[t][0];  // NF4_LEVELS[c] * scale
      const float v1 = lut[(code[t][1] >> (4 * j)) & 15u] * s[t][1];
      dst[(size_t)j * (a.K / 2)] = pack_bf16x2(v0, v1);
    }
  }
}

// With an adapter.  Wave w of a tile computes the 32 (k) x 32 (n) block
// (w / 2, w % 2) of the adapter product as (B^T A^T) with
// v_mfma_f32_32x32x16_bf16 (bf16 factors, f32 sums): with B^T as the first
// operand, lane l ends up holding row k = 32 (w / 2) + l % 32 and the 16
// columns 8 q + 4 (l / 32) + e (acc[4 q + e]) of the block, so each lane
// loads the codes of exactly those 16 (row, column) entries and adds the
// product in registers.  Adjacent lanes (rows k, k + 1) then swap half of
// their columns by DPP so that each holds whole (k, k + 1) bf16 pairs, and
// stores every pair as one dword of Wt[n][k] straight from registers (a
// half-wave writes 128 or 64 contiguous bytes of a column; no LDS tile).
// The factors' MFMA fragments are read straight from the f32 A [K][rank]
// and B [rank][N] and rounded to bf16 in registers; for rank 16 with
// 16-byte aligned factors (STAGE) the workgroup instead loads its 64 KT rows
// of A (one contiguous run) and B's 16 x 64 block once with coalesced
// 16-byte loads, rounds them into LDS and each wave reads its fragments from
// there: the per-wave strided loads fetched each factor twice per workgroup
// and more bytes of factors than the workgroup writes (config 3: 15.8 ->
// 13.6 us per expand).
//
// ROWS writes the same values row-major instead, E[k][n] ([K][N], the
// weight's own orientation: the backward's dX = dY E^T then runs as the same
// TN product as the forward), each 64 x 64 tile passed through LDS so that
// the stores are whole 128-byte row segments (8-byte stores straight from
// the MFMA layout, 32 rows x 16 bytes per instruction, took the config-3
// expand from 11.2 to 17.6 us).  With rank 0 (ROWS only) the adapter term
// is skipped and E is the dequantized weight.
template <bool DQ, bool STRIPED, int KT, int NFR, bool STAGE, bool ROWS>
__global__ __launch_bounds__(256) void expand_lora_kernel(ExpandArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int groups_k = a.tiles_k / KT;
  const int k0 = (int)(blockIdx.x % (unsigned)groups_k) * (kTile * KT);
  const int n0 = a.n_base + (int)(blockIdx.x / (unsigned)groups_k) * kTile;
  const int lane = tid & 63, wv = tid >> 6, bi = wv >> 1, bj = wv & 1, h = lane >> 5, lr = lane & 31;
  const int cb = n0 + 32 * bj;  // first column of this wave's block
  const int blk = n0 / kBlock;
  const int nf = a.rp / 16;
  static_assert(!STAGE || NFR == 1, "the staged fragments cover rank 16");

  // STAGE (rank 16, 16-byte aligned factors): the workgroup's rows of A
  // (64 KT x 16 f32, one contiguous run) and B's 16 x 64 block are loaded
  // once with coalesced 16-byte loads, before the codes
  f32x4 ga[KT], gb;
  if constexpr (STAGE) {
    const f32x4* pa = reinterpret_cast<const f32x4*>(a.la + (size_t)k0 * 16);
#pragma unroll
    for (int j = 0; j < KT; ++j) ga[j] = pa[j * 256 + tid];
    gb = *reinterpret_cast<const f32x4*>(a.lb + (size_t)(tid >> 4) * a.N + n0 + 4 * (tid & 15));
    __builtin_amdgcn_sched_barrier(0);
  }

  // codes: dword q holds columns cb + 8 q .. + 7 of the lane's row (this
  // lane uses nibbles 4 h .. 4 h + 3 of each), and the row's scale
  uint32_t cw[KT][4];
  float s[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const size_t row = (size_t)(k0 + kTile * t + 32 * bi + lr);
    size_t sidx;
    if constexpr (STRIPED) {
      const u32x2* p = reinterpret_cast<const u32x2*>(a.packed + ((size_t)(cb / 16) * a.K + row) * 8);
      const u32x2 c0 = p[0];
      const u32x2 c1 = p[a.K];  // the next stripe, same row
      cw[t][0] = c0[0];
      cw[t][1] = c0[1];
      cw[t][2] = c1[0];
      cw[t][3] = c1[1];
      sidx = (size_t)blk * a.K + row;
    } else {
      const u32x4 c = *reinterpret_cast<const u32x4*>(a.packed + row * (size_t)(a.N / 2) + cb / 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) cw[t][q] = c[q];
      sidx = row * (size_t)(a.N / kBlock) + blk;
    }
    if constexpr (DQ)
      s[t] = ((float)a.scales.dq_codes[sidx] / 255.0f) * (*a.scales.scale_of_scales);  // src/quantize.rs:349
    else
      s[t] = a.scales.absmax[sidx];
  }

  // fragments: B^T rows = columns cb + l % 32 of B, A^T columns = rows of A;
  // lane l carries adapter indices 16 f + 8 (l / 32) .. + 7
  bf16x8_t bfr[NFR];
  bf16x8_t afr[KT][NFR];
  const bool lora = a.rank > 0;  // uniform: false only for ROWS launches without an adapter
  if (!lora) {
  } else if constexpr (STAGE) {
    // bf16 A [64 KT][16] and B^T [64][16] in LDS after the wave LUTs; each
    // lane then reads its fragments as 16-byte rows
    uint32_t* sa = reinterpret_cast<uint32_t*>(smem + kLdsBytes);
    uint16_t* sb = reinterpret_cast<uint16_t*>(smem + kLdsBytes + KT * 64 * 32);
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      sa[2 * (j * 256 + tid)] = pack_bf16x2(ga[j][0], ga[j][1]);
      sa[2 * (j * 256 + tid) + 1] = pack_bf16x2(ga[j][2], ga[j][3]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) sb[(4 * (tid & 15) + e) * 16 + (tid >> 4)] = (uint16_t)pack_bf16x2(gb[e], 0.0f);
    __syncthreads();
    bfr[0] = *reinterpret_cast<const bf16x8_t*>(sb + (32 * bj + lr) * 16 + 8 * h);
#pragma unroll
    for (int t = 0; t < KT; ++t)
      afr[t][0] = *reinterpret_cast<const bf16x8_t*>(reinterpret_cast<const uint16_t*>(sa) +
                                                     (64 * t + 32 * bi + lr) * 16 + 8 * h);
  } else {
#pragma unroll
    for (int f = 0; f < NFR; ++f) {
      if (f >= nf) break;
      const int r0 = 16 * f + 8 * h;
      const size_t col = (size_t)(cb + lr);
      float bv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = r0 + e < a.rank ? a.lb[(size_t)(r0 + e) * a.N + col] : 0.0f;
      bfr[f] = __builtin_bit_cast(bf16x8_t, u32x4{pack_bf16x2(bv[0], bv[1]), pack_bf16x2(bv[2], bv[3]),
                                                  pack_bf16x2(bv[4], bv[5]), pack_bf16x2(bv[6], bv[7])});
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const size_t row = (size_t)(k0 + kTile * t + 32 * bi + lr);
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

  // one LUT copy per wave: no workgroup barrier before the decode
  float* lut = reinterpret_cast<float*>(smem + kLdsLut) + 16 * wv;
  if (lane < 16) lut[lane] = level(lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  const bool odd = (lr & 1) != 0;
  const int kpair = 16 * bi + (lr >> 1);
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    f32x16 acc = {};
#pragma unroll
    for (int f = 0; f < NFR; ++f) {
      if (!lora || f >= nf) break;
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[f], afr[t][f], acc, 0, 0, 0);
    }
    // v[4 q + e]: row k, column cb + 8 q + 4 h + e
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float w = lut[(cw[t][q] >> (16 * h + 4 * e)) & 15u] * s[t];  // NF4_LEVELS[c] * scale
        v[4 * q + e] = lora ? w + a.scaling * acc[4 * q + e] : w;
      }
    if constexpr (ROWS) {
      // the 64 x 64 tile through LDS: each wave puts its 32 x 32 block in
      // (row 32 bi + lr, columns 32 bj + 8 q + 4 h .. + 3, 8 bytes per q),
      // then each thread stores 16 bytes of rows tid / 8 and tid / 8 + 32,
      // so that every store instruction writes eight whole 128-byte rows
      unsigned char* tile = smem + kLdsBytes + (STAGE ? KT * 64 * 32 + 64 * 32 : 0);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x2*>(tile + (32 * bi + lr) * kRowPitch + (32 * bj + 8 * q + 4 * h) * 2) =
            u32x2{pack_bf16x2(v[4 * q], v[4 * q + 1]), pack_bf16x2(v[4 * q + 2], v[4 * q + 3])};
      __syncthreads();
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int r = tid / 8 + 32 * half, c = 8 * (tid % 8);
        *reinterpret_cast<u32x4*>(a.wt + (size_t)(k0 + kTile * t + r) * a.N + n0 + c) =
            *reinterpret_cast<const u32x4*>(tile + r * kRowPitch + c * 2);
      }
      __syncthreads();  // the next tile reuses the LDS tile
      continue;
    }
    // the even lane keeps columns q = 0, 1 and receives row k + 1 of them;
    // the odd lane keeps q = 2, 3 and receives row k - 1 of them; each
    // (k, k + 1) pair goes straight to Wt (for one j, 16 lanes write 64
    // consecutive bytes of one column)
    uint32_t* dst = reinterpret_cast<uint32_t*>(a.wt + (size_t)n0 * a.K + k0 + kTile * t) + kpair;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float send = odd ? v[j] : v[8 + j];
      const float keep = odd ? v[8 + j] : v[j];
      const float got = __uint_as_float(
          dpp_mov<0xB1>(__float_as_uint(send)));  // quad_perm [1,0,3,2]
      const int q = (odd ? 2 : 0) + (j >> 2), e = j & 3;
      const int col = 32 * bj + 8 * q + 4 * h + e;
      dst[(size_t)col * (a.K / 2)] = odd ? pack_bf16x2(got, keep) : pack_bf16x2(keep, got);
    }
  }
}

template <bool DQ, bool STRIPED, int KT, bool ROWS>
hipError_t launch_kt(const ExpandArgs& a, int n_count, hipStream_t stream) {
  const unsigned grid = (unsigned)((long long)(n_count / kTile) * (a.tiles_k / KT));
  if (a.rank == 0 && !ROWS)
    expand_kernel<DQ, STRIPED, KT><<<grid, 256, kLdsBytes, stream>>>(a);
  else if (a.rank == 16 && a.stage)
    expand_lora_kernel<DQ, STRIPED, KT, 1, true, ROWS>
        <<<grid, 256, kLdsBytes + KT * 64 * 32 + 64 * 32 + (ROWS ? kRowTileBytes : 0), stream>>>(a);
  else if (a.rp == 16)
    expand_lora_kernel<DQ, STRIPED, KT, 1, false, ROWS>
        <<<grid, 256, kLdsBytes + (ROWS ? kRowTileBytes : 0), stream>>>(a);
  else
    expand_lora_kernel<DQ, STRIPED, 1, kMaxRank / 16, false, ROWS>
        <<<grid, 256, kLdsBytes + (ROWS ? kRowTileBytes : 0), stream>>>(a);
  return hipGetLastError();
}

template <bool DQ, bool STRIPED, bool ROWS>
hipError_t launch_t(const ExpandArgs& a, int n_count, hipStream_t stream) {
  // four (or two) tiles per workgroup where K allows: more loads in flight
  // (with an adapter of rank <= 16, whose fragments then fit the registers)
  if (a.rank > 0 && a.rp > 16) return launch_kt<DQ, STRIPED, 1, ROWS>(a, n_count, stream);
  if (a.tiles_k % 4 == 0) return launch_kt<DQ, STRIPED, 4, ROWS>(a, n_count, stream);
  if (a.tiles_k % 2 == 0) return launch_kt<DQ, STRIPED, 2, ROWS>(a, n_count, stream);
  return launch_kt<DQ, STRIPED, 1, ROWS>(a, n_count, stream);
}

template <bool ROWS>
hipError_t launch_layout(const ExpandArgs& a, bool dq, bool striped, int n_count, hipStream_t stream) {
  if (dq) return striped ? launch_t<true, true, ROWS>(a, n_count, stream) : launch_t<true, false, ROWS>(a, n_count, stream);
  return striped ? launch_t<false, true, ROWS>(a, n_count, stream) : launch_t<false, false, ROWS>(a, n_count, stream);
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

namespace {

// The arguments of one expand launch over columns [n_begin, n_end).
bool expand_args(const uint8_t* packed, const ScalesArg& scales, int K, int N, const float* lora_a,
                 const float* lora_b, int rank, float scaling, int n_begin, int n_end, uint16_t* out, ExpandArgs* a) {
  if (!expand_supported(K, N, rank) || (rank > 0 && (!lora_a || !lora_b)) || n_begin < 0 || n_end > N ||
      n_begin % kTile != 0 || n_end % kTile != 0 || n_begin >= n_end)
    return false;
  if ((long long)(K / kTile) * ((n_end - n_begin) / kTile) > 0x7fffffffLL) return false;
  *a = ExpandArgs{};
  a->packed = packed;
  a->scales = scales;
  a->K = K;
  a->N = N;
  a->la = lora_a;
  a->lb = lora_b;
  a->la_vec = rank % 8 == 0 && (reinterpret_cast<uintptr_t>(lora_a) & 15u) == 0;
  a->stage = rank == 16 && (reinterpret_cast<uintptr_t>(lora_a) & 15u) == 0 &&
             (reinterpret_cast<uintptr_t>(lora_b) & 15u) == 0;
  a->rank = rank;
  a->rp = rank <= 16 ? 16 : rank <= 32 ? 32 : 64;
  a->scaling = scaling;
  a->wt = out;
  a->tiles_k = K / kTile;
  a->n_base = n_begin;
  return true;
}

}  // namespace

hipError_t launch_expand_cols(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                              const float* lora_a, const float* lora_b, int rank, float scaling, int n_begin, int n_end,
                              uint16_t* wt, hipStream_t stream) {
  ExpandArgs a;
  if (!expand_args(packed, scales, K, N, lora_a, lora_b, rank, scaling, n_begin, n_end, wt, &a))
    return hipErrorInvalidValue;
  return launch_layout<false>(a, scales.kind == kScalesDQ, striped, n_end - n_begin, stream);
}

hipError_t launch_expand_rows_bf16(const uint8_t* packed, const ScalesArg& scales, int K, int N, bool striped,
                                   const float* lora_a, const float* lora_b, int rank, float scaling, uint16_t* e,
                                   hipStream_t stream) {
  ExpandArgs a;
  if (!expand_args(packed, scales, K, N, lora_a, lora_b, rank, scaling, 0, N, e, &a)) return hipErrorInvalidValue;
  return launch_layout<true>(a, scales.kind == kScalesDQ, striped, N, stream);
}

}  // namespace unifur
