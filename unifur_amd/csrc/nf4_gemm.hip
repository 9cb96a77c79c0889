// nf4_gemm.hip -- MFMA bf16 prefill GEMM with the NF4 weight dequantized
// into LDS, and the scaled LoRA update fused into the epilogue.
//
// Y[M, N] = X[M, K] deq(W)[K, N] (+ bias) (+ scaling * (X A)[M, r] B[r, N]),
// X bf16 row-major, W the reference's packed [d_in, d_out] NF4 weight
// (src/qwennet.rs:161-241 for the base, src/qwennet.rs:325-345 and
// src/quantize.rs:619-624 for the adapter).  The dequantized weight value
// NF4_LEVELS[c] * scale is the reference's f32 value (src/quantize.rs:362),
// rounded to bf16 for the MFMA; products accumulate in f32.
//
// Tiling.  A 512-thread workgroup computes a 256 x 128 output tile, K in
// steps of 64.  It is warp-specialised: four MFMA waves (one per SIMD) each
// own 64 rows x 128 columns (2 x 4 MFMA 32x32x16 tiles, f32 accumulators),
// copy their own X rows into LDS with coalesced buffer_load ... lds copies
// (three stages, two steps ahead), read operand fragments one k16 slice
// ahead of the MFMAs and issue the MFMAs; four producer waves (one per SIMD
// beside an MFMA wave) expand the NF4 codes (byte LUT -> level pair, x
// block scale, -> bf16) two steps ahead into a three-buffer W tile ring
// stored [n][k], so that every MFMA operand fetch is one 16-byte ds_read.
// Their VALU / LDS work overlaps the MFMAs on the same SIMD; one workgroup
// barrier per step (an LDS-only barrier: no wait for outstanding global
// loads) hands the W buffers over.  Both tiles use a 16-byte-chunk XOR
// swizzle, chunk ^ ((row % 8) ^ (row / 8 % 8)), which makes the operand
// reads (8 consecutive rows, one chunk) conflict-free.
#include "nf4_gemm.hpp"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace unifur {
namespace {

constexpr int kBM = 256, kBN = 128, kBK = 64;
constexpr int kGemmThreads = 512;  // 4 MFMA waves + 4 producer waves
constexpr int kBTileBytes = kBN * kBK * 2;       // dequantized bf16 W tile: 16 KiB
constexpr int kATileBytes = kBM * kBK * 2;       // X tile: 32 KiB (8 KiB per wave)
constexpr int kAStages = 3;
constexpr int kLdsA = 0;                         // kAStages buffers
constexpr int kBStages = 3;
constexpr int kLdsB = kAStages * kATileBytes;    // kBStages buffers
// Level lookup of the W-dequantizing waves (UNIFUR_GEMM_LUT): 0 = one byte
// LUT (256 x {level lo, level hi}), 1 = four copies of it (lane % 4 picks
// one, fewer bank conflicts), 2 = a 16-entry level table read per nibble
// (64 lanes meet at most 16 addresses in 16 banks: broadcast, no conflicts).
#ifndef UNIFUR_GEMM_LUT
#define UNIFUR_GEMM_LUT 0
#endif
constexpr int kLutMode = UNIFUR_GEMM_LUT;
static_assert(kLutMode >= 0 && kLutMode <= 2, "UNIFUR_GEMM_LUT");
constexpr int kLutBytes = kLutMode == 1 ? 4 * 256 * 8 : kLutMode == 2 ? 16 * 4 : 256 * 8;
constexpr int kLdsLut = kLdsB + kBStages * kBTileBytes;  // level LUT
constexpr int kLdsDq = kLdsLut + kLutBytes;      // DQ scale LUTs, 256 x f32 per weight (two in PAIR mode)
constexpr size_t kGemmSmem = kLdsDq + 2 * 256 * 4;  // 148 KiB: one workgroup per CU

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) const f32x2 lds_f32x2_c;

struct GemmArgs {
  const uint16_t* x;  // [M, K] bf16
  const uint8_t* packed;
  ScalesArg scales;
  int M, K, N;
  const float* bias;     // [N] or null
  const uint16_t* lora_xa;  // bf16 [M, lora_pad]: scaling * (x A), zero past lora_rank; or null
  const uint16_t* lora_bt;  // bf16 [N, lora_pad]: B transposed, zero past lora_rank
  int lora_rank, lora_pad;
  void* y;  // [M, N] f32 or bf16
  int y_bf16;
  int y_aligned;  // y 16-byte aligned: the epilogue stores 4 outputs at once
  int tiles_n;  // N / kBN (N / 64 in PAIR mode)
  // split-K: k_splits workgroups per output tile, each over k_steps K steps
  // (the last over what is left), writing its raw f32 sums to partials
  // [k_splits][M][ldy] (bias, adapter and rounding come in the reduction)
  int k_splits, k_steps;
  float* partials;
  int ldy;  // row stride of the split-K partials: N, or 2 N in PAIR mode (gate columns, then up)
  // PAIR mode (the SwiGLU gate/up pair over one X): the second weight (up),
  // same shape, layout and scale kind as the first (gate).  A tile holds 64
  // columns of each -- W tile columns 0-63 gate, 64-127 up -- and stores
  // silu(gate x) * (up x) for its 64 columns.
  const uint8_t* packed2;
  ScalesArg scales2;
  // tiles of this launch: tile_count tiles from tile_begin in the (m, n)
  // row-major tile order (tile_count 0: all of them)
  int tile_begin, tile_count;
};

// silu(z) * u, the middle of QwenMlp::forward (src/qwennet.rs:816-819,
// src/tensor_ext.rs:87-90), the expression the elementwise kernels use.
__device__ __forceinline__ float silu_times(float z, float u) { return (z * (1.0f / (1.0f + __expf(-z)))) * u; }

// 16-byte chunk swizzle of a 128-byte tile row (8 chunks).
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row & 7) ^ ((row >> 3) & 7)); }

__device__ __forceinline__ uint32_t lds_addr(int base, int row, int chunk) {
  return (uint32_t)(base + row * (kBK * 2) + swz(row, chunk) * 16);
}

// X tile of one K step, copied by each wave for its own 64 rows straight
// from global memory into its LDS region (buffer_load ... lds): 8 coalesced
// 1 KiB copies of 8 rows x 128 bytes.  Lane l of copy p writes LDS slot l,
// i.e. row 8 p + l / 8, physical chunk l % 8, so it fetches the logical chunk
// that the swizzle puts there.  Rows past M read as zero (buffer bound).
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void load_a(__amdgpu_buffer_rsrc_t xr, int K, int row0, int k0, int abase, int lane) {
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int r = 8 * p + (lane >> 3);
    const int c = swz(r, lane & 7);  // swz is an involution on the chunk index
    const uint32_t off = ((uint32_t)(row0 + r) * (uint32_t)K + (uint32_t)(k0 + 8 * c)) * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(size_t)(abase + p * 1024), 16, off, 0, 0, 0);
  }
}

// NF4 codes and block scales of one K step for producer thread d (0..255):
// stripe st = d / 32 of the tile (columns n0 + 16 st .. + 15) at rows
// k0 + 2 (d % 32) and the next -- 8 code bytes of each row.  The 256 threads
// cover the 64 x 128 W tile once.
struct BStep {
  uint32_t code[4];   // row 0 bytes 0-3, 4-7, then row 1
  uint32_t scale[2];  // f32 bits, or u8 DQ codes (striped DQ: both rows in scale[0])
};

// The weight a producer thread reads: its codes, scales and the first of its
// 16 columns.
struct BSrc {
  const uint8_t* packed;
  ScalesArg scales;
  int n;
};

template <bool DQ, bool STRIPED>
__device__ __forceinline__ void load_b(BStep& B, const GemmArgs& g, const BSrc& w, int k0, int d) {
  const int n = w.n, k = k0 + 2 * (d & 31);
  if constexpr (STRIPED) {
    // stripe n / 16 holds 8 bytes per row, rows consecutive
    const uint8_t* cp = w.packed + ((size_t)(n / 16) * g.K + k) * 8;
    const u32x2 r0 = *reinterpret_cast<const u32x2*>(cp);
    const u32x2 r1 = *reinterpret_cast<const u32x2*>(cp + 8);
    B.code[0] = r0.x;
    B.code[1] = r0.y;
    B.code[2] = r1.x;
    B.code[3] = r1.y;
    // block-major scales: rows k, k + 1 of block n / 64 are consecutive (k even)
    const size_t blk = (size_t)(n / kBlock) * g.K + k;
    if constexpr (DQ) {
      // the aligned dword holding both rows' u8 codes (bytes 2 (d % 2), + 1:
      // blk % 4 == k % 4 == 2 (d % 2)); a dword load leaves no zero-extension
      // for the compiler to place away from the decode
      B.scale[0] = *reinterpret_cast<const uint32_t*>(w.scales.dq_codes + (blk & ~size_t{3}));
      B.scale[1] = 0u;
    } else {
      const u32x2 s2 = *reinterpret_cast<const u32x2*>(w.scales.absmax + blk);
      B.scale[0] = s2.x;
      B.scale[1] = s2.y;
    }
  } else {
    const size_t row_bytes = (size_t)g.N / 2, bpr = (size_t)g.N / kBlock;
    const uint8_t* cp = w.packed + (size_t)k * row_bytes + n / 2;
    const u32x2 r0 = *reinterpret_cast<const u32x2*>(cp);
    const u32x2 r1 = *reinterpret_cast<const u32x2*>(cp + row_bytes);
    B.code[0] = r0.x;
    B.code[1] = r0.y;
    B.code[2] = r1.x;
    B.code[3] = r1.y;
    const size_t blk = (size_t)k * bpr + n / kBlock;
    if constexpr (DQ) {
      B.scale[0] = w.scales.dq_codes[blk];
      B.scale[1] = w.scales.dq_codes[blk + bpr];
    } else {
      B.scale[0] = __float_as_uint(w.scales.absmax[blk]);
      B.scale[1] = __float_as_uint(w.scales.absmax[blk + bpr]);
    }
  }
}

// Codes -> dequantized bf16 W tile [n][k] in LDS buffer buf: byte j of a row
// holds columns 2j (low nibble) and 2j + 1; one byte-LUT lookup gives both
// levels, each times its row's block scale (one f32 multiply, as the
// reference's dequantize), rounded to bf16, and the (k, k + 1) pair of a
// column is one 4-byte LDS store.
template <bool DQ, bool STRIPED>
__device__ __forceinline__ void store_b_at(const BStep& B, unsigned char* smem, int ring, int lut_off, int dq_off,
                                           int buf, int d, int dq_table) {
  const int st = d >> 5, rp = d & 31;
  const float* dq_lut = reinterpret_cast<const float*>(smem + dq_off + dq_table * 1024);
  float s0, s1;
  if constexpr (DQ && STRIPED) {
    const int sh = 16 * (d & 1);
    s0 = dq_lut[(B.scale[0] >> sh) & 0xffu];
    s1 = dq_lut[(B.scale[0] >> (sh + 8)) & 0xffu];
  } else if constexpr (DQ) {
    s0 = dq_lut[B.scale[0] & 0xffu];
    s1 = dq_lut[B.scale[1] & 0xffu];
  } else {
    s0 = __uint_as_float(B.scale[0]);
    s1 = __uint_as_float(B.scale[1]);
  }
  const int base = ring + buf * kBTileBytes;
  const int chunk = rp >> 2;                   // k = 2 rp lies in 16-byte chunk rp / 4 of a row
  const uint32_t within = (uint32_t)(rp & 3) * 4u;
  // all 16 lookups first, so that one LDS latency covers them (a producer
  // wave has its SIMD to itself beside an MFMA wave: nothing else hides it)
  f32x2 l[2][8];
  if constexpr (kLutMode == 2) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint32_t w = B.code[2 * r + (j >> 2)], sh = 8 * (j & 3);
        l[r][j].x = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
            (size_t)(lut_off + (((w >> sh) & 0xfu) << 2)));
        l[r][j].y = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
            (size_t)(lut_off + (((w >> (sh + 4)) & 0xfu) << 2)));
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 32, 1);  // the 32 level reads
  } else {
    const uint32_t copy = kLutMode == 1 ? (uint32_t)(d & 3) * 2048u : 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint32_t byte = (B.code[2 * r + (j >> 2)] >> (8 * (j & 3))) & 0xffu;
        l[r][j] = *reinterpret_cast<lds_f32x2_c*>((size_t)(lut_off + copy + byte * 8));
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 1);  // the 16 LUT reads
  }
  __builtin_amdgcn_sched_group_barrier(0x002, 64, 1);  // then VALU
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t even = pack_bf16x2(l[0][j].x * s0, l[1][j].x * s1);  // column 2j, rows k and k + 1
    const uint32_t odd = pack_bf16x2(l[0][j].y * s0, l[1][j].y * s1);   // column 2j + 1
    const int n = 16 * st + 2 * j;
    *reinterpret_cast<lds_u32*>((size_t)(lds_addr(base, n, chunk) + within)) = even;
    *reinterpret_cast<lds_u32*>((size_t)(lds_addr(base, n + 1, chunk) + within)) = odd;
  }
}

// The same tile in 8-byte stores: lanes d and d ^ 1 (row pairs 2i and 2i + 1
// of one stripe: rows 4i .. 4i + 3) swap half their codes and their row
// scales by DPP, so that the even lane holds columns 0-7 and the odd lane
// columns 8-15 of all four rows; each of a lane's 8 columns then has its 4
// consecutive k in one bf16 quad, one ds_write_b64 (8 stores per step
// instead of 16 dword stores).
#ifndef UNIFUR_GEMM_STORE64
#define UNIFUR_GEMM_STORE64 2
#endif
__device__ __forceinline__ uint32_t swap_lane_pair(uint32_t v) {
  return dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
}

template <bool DQ, bool STRIPED>
__device__ __forceinline__ void store_b64(const BStep& B, unsigned char* smem, int buf, int d, int dq_table) {
  static_assert(kLutMode == 0, "the paired store reads the one-copy byte LUT");
  const int st = d >> 5, rp = d & 31;
  const bool odd = (d & 1) != 0;
  const float* dq_lut = reinterpret_cast<const float*>(smem + kLdsDq + dq_table * 1024);
  float s0, s1;  // this lane's rows 2 rp, 2 rp + 1
  if constexpr (DQ && STRIPED) {
    const int sh = 16 * (d & 1);
    s0 = dq_lut[(B.scale[0] >> sh) & 0xffu];
    s1 = dq_lut[(B.scale[0] >> (sh + 8)) & 0xffu];
  } else if constexpr (DQ) {
    s0 = dq_lut[B.scale[0] & 0xffu];
    s1 = dq_lut[B.scale[1] & 0xffu];
  } else {
    s0 = __uint_as_float(B.scale[0]);
    s1 = __uint_as_float(B.scale[1]);
  }
  // even lane keeps bytes 0-3 (columns 0-7) and sends bytes 4-7; odd the reverse
  const uint32_t r0 = swap_lane_pair(odd ? B.code[0] : B.code[1]);
  const uint32_t r1 = swap_lane_pair(odd ? B.code[2] : B.code[3]);
  const float t0 = __uint_as_float(swap_lane_pair(__float_as_uint(s0)));
  const float t1 = __uint_as_float(swap_lane_pair(__float_as_uint(s1)));
  // rows 4i .. 4i + 3 (i = rp / 2): the even lane's own two, then its partner's
  const uint32_t w[4] = {odd ? r0 : B.code[0], odd ? r1 : B.code[2], odd ? B.code[1] : r0, odd ? B.code[3] : r1};
  const float sc[4] = {odd ? t0 : s0, odd ? t1 : s1, odd ? s0 : t0, odd ? s1 : t1};
  if constexpr (UNIFUR_GEMM_STORE64 == 2) {
    // second exchange, lanes d and d ^ 2 (rows 8g .. 8g + 3 and 8g + 4 ..
    // 8g + 7, g = rp / 4): each keeps 4 of its 8 columns (the u16 half e =
    // bit 1 of d of every row dword) and takes the partner's rows of them, so
    // a lane holds 8 rows x 4 columns and a column's 8 k are one 16-byte store
    const uint32_t e = (uint32_t)(d >> 1) & 1u;
    const uint32_t ks = (2u * e) | ((2u * e + 1u) << 8) | ((4u + 2u * e) << 16) | ((5u + 2u * e) << 24);
    const uint32_t ss = ks ^ 0x02020202u;  // the other half
    const uint32_t k01 = __builtin_amdgcn_perm(w[1], w[0], ks), k23 = __builtin_amdgcn_perm(w[3], w[2], ks);
    const uint32_t r01 = dpp_mov<0x4E>(__builtin_amdgcn_perm(w[1], w[0], ss));
    const uint32_t r23 = dpp_mov<0x4E>(__builtin_amdgcn_perm(w[3], w[2], ss));
    float so[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      so[q] = __uint_as_float(dpp_mov<0x4E>(__float_as_uint(sc[q])));
    // rows 8g + 2p, 8g + 2p + 1 in dword p (low, high u16)
    const uint32_t D[4] = {e ? r01 : k01, e ? r23 : k23, e ? k01 : r01, e ? k23 : r23};
    float s8[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      s8[q] = e ? so[q] : sc[q];
      s8[4 + q] = e ? sc[q] : so[q];
    }
    f32x2 l8[8][2];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr)
#pragma unroll
      for (int b = 0; b < 2; ++b)
        l8[rr][b] = *reinterpret_cast<lds_f32x2_c*>(
            (size_t)(kLdsLut + ((D[rr >> 1] >> (16 * (rr & 1) + 8 * b)) & 0xffu) * 8));
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 1);  // the 16 LUT reads
    __builtin_amdgcn_sched_group_barrier(0x002, 64, 1);  // then VALU
    const int base = kLdsB + buf * kBTileBytes;
    const int g8 = rp >> 2;                                   // chunk: k 8 g8 .. 8 g8 + 7
    const int nc = 16 * st + 8 * (d & 1) + 4 * (int)e;        // first of the lane's 4 columns
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      u32x4 lo, hi;  // columns 2b (level .x) and 2b + 1 (.y)
      lo.x = pack_bf16x2(l8[0][b].x * s8[0], l8[1][b].x * s8[1]);
      lo.y = pack_bf16x2(l8[2][b].x * s8[2], l8[3][b].x * s8[3]);
      lo.z = pack_bf16x2(l8[4][b].x * s8[4], l8[5][b].x * s8[5]);
      lo.w = pack_bf16x2(l8[6][b].x * s8[6], l8[7][b].x * s8[7]);
      hi.x = pack_bf16x2(l8[0][b].y * s8[0], l8[1][b].y * s8[1]);
      hi.y = pack_bf16x2(l8[2][b].y * s8[2], l8[3][b].y * s8[3]);
      hi.z = pack_bf16x2(l8[4][b].y * s8[4], l8[5][b].y * s8[5]);
      hi.w = pack_bf16x2(l8[6][b].y * s8[6], l8[7][b].y * s8[7]);
      *reinterpret_cast<lds_u32x4*>((size_t)lds_addr(base, nc + 2 * b, g8)) = lo;
      *reinterpret_cast<lds_u32x4*>((size_t)lds_addr(base, nc + 2 * b + 1, g8)) = hi;
    }
    return;
  }
  f32x2 l[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      l[q][j] = *reinterpret_cast<lds_f32x2_c*>((size_t)(kLdsLut + ((w[q] >> (8 * j)) & 0xffu) * 8));
  __builtin_amdgcn_sched_group_barrier(0x100, 16, 1);  // the 16 LUT reads
  __builtin_amdgcn_sched_group_barrier(0x002, 64, 1);  // then VALU
  const int base = kLdsB + buf * kBTileBytes;
  const int k4 = 4 * (rp >> 1);                       // first of the 4 rows (k of the tile)
  const int n0 = 16 * st + 8 * (d & 1);               // first of the lane's 8 columns
  const uint32_t within = (uint32_t)(k4 & 7) * 2u;    // byte offset of k4 in its 16-byte chunk
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x2 even = {pack_bf16x2(l[0][j].x * sc[0], l[1][j].x * sc[1]),
                        pack_bf16x2(l[2][j].x * sc[2], l[3][j].x * sc[3])};  // column 2j
    const u32x2 oddc = {pack_bf16x2(l[0][j].y * sc[0], l[1][j].y * sc[1]),
                        pack_bf16x2(l[2][j].y * sc[2], l[3][j].y * sc[3])};  // column 2j + 1
    *reinterpret_cast<lds_u32x2*>((size_t)(lds_addr(base, n0 + 2 * j, k4 >> 3) + within)) = even;
    *reinterpret_cast<lds_u32x2*>((size_t)(lds_addr(base, n0 + 2 * j + 1, k4 >> 3) + within)) = oddc;
  }
}

template <bool DQ, bool STRIPED>
__device__ __forceinline__ void store_b(const BStep& B, unsigned char* smem, int buf, int d, int dq_table) {
  if constexpr (UNIFUR_GEMM_STORE64 && kLutMode == 0)
    store_b64<DQ, STRIPED>(B, smem, buf, d, dq_table);
  else
    store_b_at<DQ, STRIPED>(B, smem, kLdsB, kLdsLut, kLdsDq, buf, d, dq_table);
}

// TRANS (dX = dY W^T over a striped weight W [d_in][d_out]): the tile's 128
// outputs are W rows w.n .. w.n + 127 and a K step is W columns k0 .. k0 +
// 63, one block.  Producer thread d takes stripe k0 / 16 + d / 64 (16
// columns) of rows w.n + 2 (d % 64) and the next -- 8 code bytes each,
// consecutive in the stripe -- and the two rows' scales of that block
// (block-major, also consecutive); g.N is d_in here.
template <bool DQ>
__device__ __forceinline__ void load_bt(BStep& B, const GemmArgs& g, const BSrc& w, int k0, int d) {
  const int r = w.n + 2 * (d & 63);
  const uint8_t* cp = w.packed + ((size_t)(k0 / 16 + (d >> 6)) * g.N + r) * 8;
  const u32x2 r0 = *reinterpret_cast<const u32x2*>(cp);
  const u32x2 r1 = *reinterpret_cast<const u32x2*>(cp + 8);
  B.code[0] = r0.x;
  B.code[1] = r0.y;
  B.code[2] = r1.x;
  B.code[3] = r1.y;
  const size_t blk = (size_t)(k0 / kBlock) * g.N + r;
  if constexpr (DQ) {
    // the aligned dword holding both rows' u8 codes: blk % 4 == r % 4 == 2 (d % 2)
    B.scale[0] = *reinterpret_cast<const uint32_t*>(w.scales.dq_codes + (blk & ~size_t{3}));
    B.scale[1] = 0u;
  } else {
    const u32x2 s2 = *reinterpret_cast<const u32x2*>(w.scales.absmax + blk);
    B.scale[0] = s2.x;
    B.scale[1] = s2.y;
  }
}

// ... and its tile rows 2 (d % 64), + 1: byte j of a row holds columns 2j
// (low nibble) and 2j + 1, i.e. k and k + 1 of the tile row, so each level
// pair times the row's scale is one bf16 dword and the 16 values of a row
// are the two 16-byte chunks 2 (d / 64), + 1 of that row.
template <bool DQ>
__device__ __forceinline__ void store_bt(const BStep& B, unsigned char* smem, int buf, int d) {
  static_assert(kLutMode == 0, "the transposed producer reads the one-copy byte LUT");
  const float* dq_lut = reinterpret_cast<const float*>(smem + kLdsDq);
  float sc[2];
  if constexpr (DQ) {
    const int sh = 16 * (d & 1);
    sc[0] = dq_lut[(B.scale[0] >> sh) & 0xffu];
    sc[1] = dq_lut[(B.scale[0] >> (sh + 8)) & 0xffu];
  } else {
    sc[0] = __uint_as_float(B.scale[0]);
    sc[1] = __uint_as_float(B.scale[1]);
  }
  f32x2 l[2][8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t byte = (B.code[2 * r + (j >> 2)] >> (8 * (j & 3))) & 0xffu;
      l[r][j] = *reinterpret_cast<lds_f32x2_c*>((size_t)(kLdsLut + byte * 8));
    }
  __builtin_amdgcn_sched_group_barrier(0x100, 16, 1);  // the 16 LUT reads first
  __builtin_amdgcn_sched_group_barrier(0x002, 64, 1);  // then VALU
  const int base = kLdsB + buf * kBTileBytes, row = 2 * (d & 63), ch = 2 * (d >> 6);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = pack_bf16x2(l[r][j].x * sc[r], l[r][j].y * sc[r]);
    *reinterpret_cast<lds_u32x4*>((size_t)lds_addr(base, row + r, ch)) = u32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<lds_u32x4*>((size_t)lds_addr(base, row + r, ch + 1)) = u32x4{v[4], v[5], v[6], v[7]};
  }
}

__device__ __forceinline__ bf16x8 read_frag(int base, int row, int chunk) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<lds_u32x4*>((size_t)lds_addr(base, row, chunk)));
}

// One K step: the wave's 64 x 128 tile as 2 x 4 32x32x16 MFMA tiles over
// four k16 slices, A fragments from the wave's LDS region at abase and B
// fragments from the W tile at bbase.  The k order inside a step is permuted
// the same way for both operands: lane l's slice kk is chunk 4 (l / 32) + kk.
// The fragments of slice kk + 1 are read while slice kk's MFMAs run.
struct Frags {
  bf16x8 a[2], b[4];
};

__device__ __forceinline__ void read_frags(Frags& F, int abase, int bbase, int kk, int lane) {
  const int ch = 4 * (lane >> 5) + kk;
#pragma unroll
  for (int i = 0; i < 2; ++i) F.a[i] = read_frag(abase, 32 * i + (lane & 31), ch);
#pragma unroll
  for (int j = 0; j < 4; ++j) F.b[j] = read_frag(bbase, 32 * j + (lane & 31), ch);
}

// The 8 MFMAs of one k16 slice.  The scheduling groups put the fragment
// reads the caller issued just before (6 ds_read_b128, the next slice's)
// ahead of these MFMAs, so that their LDS latency hides behind them.
__device__ __forceinline__ void mma_frags(f32x16 (&acc)[2][4], const Frags& F) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.a[i], F.b[j], acc[i][j], 0, 0, 0);
  __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // DS reads first
  __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // then the MFMAs
}

// vmcnt(n): wait until at most n vector-memory loads of this wave are in
// flight (they complete in issue order).
#define UNIFUR_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

// Workgroup barrier for LDS hand-offs only: this wave's LDS operations
// complete (lgkmcnt(0)), then s_barrier.  Unlike __syncthreads() it does not
// wait for the wave's vector-memory loads, so the X copies and code loads
// issued steps ahead stay in flight across it.  The signal fences keep the
// compiler from moving memory operations across the barrier, the scheduling
// barriers any instruction (a later step's code decoding hoisted above it
// would wait for that step's loads here).
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt 63, expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The end of a tile: the adapter's (x A) B added on MFMA (LORA), then the
// store epilogue through this wave's 16 KiB of LDS staging -- rows 0-15 of
// each 32-row half at stage0, rows 16-31 at stage1, 512 bytes a row.
template <bool YBF16, bool LORA, bool PAIR>
__device__ __forceinline__ void finish_tile(const GemmArgs& g, f32x16 (&acc)[2][4], void* yout, int row0, int n0,
                                            int lane, uint32_t stage0, uint32_t stage1) {
  if constexpr (LORA) {
    // acc += xa[rows, r] . B[r, cols] (xa already scaled), one 32x32x16 MFMA
    // per tile and 16 adapter columns; both operands are bf16 laid out so
    // that each fragment is one 16-byte load (columns past the rank are zero).
    const int kr = (lane >> 5) * 8;
    for (int r0 = 0; r0 < g.lora_pad; r0 += 16) {
      bf16x8 bfr[4], af[2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + 32 * j + (lane & 31);
        bfr[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(g.lora_bt + (size_t)n * g.lora_pad + r0 + kr));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int m = row0 + 32 * i + (lane & 31);
        af[i] = m < g.M ? __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(g.lora_xa + (size_t)m * g.lora_pad + r0 + kr))
                        : bf16x8{};
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue, through this wave's own X-stage chunks of stages 0 and 1 (its
  // copies all landed and its reads completed in the last step; no other
  // wave touches them).  acc[i][j][4 a + e] is C[row 32 i + 8 a + 4 (lane /
  // 32) + e][col 32 j + lane % 32]; each half i (32 rows) of the wave's tile
  // is staged as f32 -- row r at chunk r / 16, byte (r % 16) * 512 +
  // (4 c ^ 128 * (r / 4 % 2)), so that the two row groups of a store land in
  // different bank halves -- then read back row-contiguous: lane l takes
  // columns 4 (l % 32) .. + 3 of row 2 q + l / 32 and writes them as one
  // 16-byte (f32) or 8-byte (bf16) store, the bias added.
  {
    const int cq = 4 * (lane & 31);
    float bias4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (g.bias) {
#pragma unroll
      for (int t2 = 0; t2 < 4; ++t2) bias4[t2] = g.bias[n0 + cq + t2];
    }
    auto stage_off = [&](int r, int c) -> uint32_t {
      return (r < 16 ? stage0 : stage1) + (uint32_t)((r & 15) * 512) +
             (((uint32_t)c * 4u) ^ ((uint32_t)((r >> 2) & 1) << 7));
    };
    if constexpr (PAIR && YBF16) {
      // silu(gate x) * (up x): acc[i][j] (gate columns 32 j ..) and
      // acc[i][j + 2] (up, the same columns) hold their elements in the same
      // lanes, so the product forms in registers; the 32 x 64 block of each
      // half i is staged as above, then read back 16 lanes per row (columns
      // 4 (l % 16) .. + 3 of row 4 q + l / 16) and stored as four bf16
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              *reinterpret_cast<__attribute__((address_space(3))) float*>(
                  (size_t)stage_off(8 * a4 + 4 * (lane >> 5) + e, 32 * j + (lane & 31))) =
                  silu_times(acc[i][j][4 * a4 + e], acc[i][j + 2][4 * a4 + e]);
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        const int c4 = 4 * (lane & 15);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int r = 4 * q + (lane >> 4);
          const int m = row0 + 32 * i + r;
          const f32x4 v = *reinterpret_cast<__attribute__((address_space(3))) const f32x4*>((size_t)stage_off(r, c4));
          if (m < g.M) {
            const u32x2 o = {pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
            uint16_t* p = reinterpret_cast<uint16_t*>(yout) + (size_t)m * g.N + n0 + c4;
            if (g.y_aligned) {
              *reinterpret_cast<u32x2*>(p) = o;
            } else {
              p[0] = (uint16_t)(o.x & 0xffffu);
              p[1] = (uint16_t)(o.x >> 16);
              p[2] = (uint16_t)(o.y & 0xffffu);
              p[3] = (uint16_t)(o.y >> 16);
            }
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();  // the next half reuses the chunks
      }
      return;
    }
    // columns of this lane's four outputs: PAIR split-K partials put the
    // gate columns at n0 .. and the up columns at N + n0 .. of a 2 N row
    const int col = PAIR && cq >= 64 ? g.N + n0 + cq - 64 : n0 + cq;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *reinterpret_cast<__attribute__((address_space(3))) float*>(
                (size_t)stage_off(8 * a4 + 4 * (lane >> 5) + e, 32 * j + (lane & 31))) = acc[i][j][4 * a4 + e];
      __builtin_amdgcn_s_waitcnt(0xc07f);  // a wave's LDS operations complete in order; be explicit
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int r = 2 * q + (lane >> 5);
        const int m = row0 + 32 * i + r;
        const f32x4 v = *reinterpret_cast<__attribute__((address_space(3))) const f32x4*>((size_t)stage_off(r, cq));
        if (m < g.M) {
          const size_t idx = (size_t)m * g.ldy + col;
          const float y0 = v.x + bias4[0], y1 = v.y + bias4[1], y2 = v.z + bias4[2], y3 = v.w + bias4[3];
          if constexpr (YBF16) {
            const u32x2 o = {pack_bf16x2(y0, y1), pack_bf16x2(y2, y3)};
            if (g.y_aligned) {
              *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(yout) + idx) = o;
            } else {
              uint16_t* p = reinterpret_cast<uint16_t*>(yout) + idx;
              p[0] = (uint16_t)(o.x & 0xffffu);
              p[1] = (uint16_t)(o.x >> 16);
              p[2] = (uint16_t)(o.y & 0xffffu);
              p[3] = (uint16_t)(o.y >> 16);
            }
          } else {
            float* p = reinterpret_cast<float*>(yout) + idx;
            if (g.y_aligned) {
              *reinterpret_cast<f32x4*>(p) = f32x4{y0, y1, y2, y3};
            } else {
              p[0] = y0;
              p[1] = y1;
              p[2] = y2;
              p[3] = y3;
            }
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();  // the next half reuses the chunks
    }
  }
}

// Workgroup tile 256 x 128, warp-specialised: waves 0-3 ("MFMA waves") own
// rows 64 w .. + 63 and all 128 columns; each copies its own X rows into its
// LDS region (buffer_load ... lds, two steps ahead, three stages), reads
// fragments and issues MFMAs, the next slice's fragments read while the
// current slice's MFMAs run (across steps too: the next step's first slice
// is read during the current step's last).  Waves 4-7 ("producer waves", one
// per SIMD beside an MFMA wave) dequantize the W tile two steps ahead into a
// three-buffer ring, from codes loaded four steps ahead in registers, so
// that their VALU / LDS work overlaps the MFMAs on the same SIMD.  One
// workgroup barrier per K step hands the W buffers over: barrier s + 1 comes
// after the producers wrote step s + 2 and the MFMA waves read the last of
// step s; X needs none (each MFMA wave reads only the rows it copied itself,
// after waiting for its own copies).
template <bool DQ, bool YBF16, bool LORA, bool STRIPED, bool PAIR, bool TRANS = false>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs g) {
  static_assert(!(PAIR && LORA), "the SwiGLU pair has no adapter");
  static_assert(!TRANS || (STRIPED && !PAIR), "the transposed weight is striped, one weight");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int w4 = wave & 3;  // MFMA wave index (waves 0-3)

  // XCD-aware tile order: workgroup b runs on XCD b % 8; each XCD takes a
  // contiguous run of tiles in row-major (m, n) order, so the workgroups
  // sharing an X row band share that XCD's L2.
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int tb = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
  const int split = tb % g.k_splits, t = g.tile_begin + tb / g.k_splits;
  const int m0 = (t / g.tiles_n) * kBM, n0 = (t % g.tiles_n) * (PAIR ? kBN / 2 : kBN);
  const int row0 = m0 + 64 * w4;
  const int kb = split * g.k_steps;  // this workgroup's first K step
  const int kbase = kb * kBK;        // ... as a column of X / row of W
  void* const yout = g.k_splits > 1 ? static_cast<void*>(g.partials + (size_t)split * g.M * g.ldy) : g.y;

  if (tid < 256) {
    float* lut = reinterpret_cast<float*>(smem + kLdsLut);
    if constexpr (kLutMode == 2) {
      if (tid < 16) lut[tid] = level(tid);
    } else {
#pragma unroll
      for (int c = 0; c < (kLutMode == 1 ? 4 : 1); ++c) {
        lut[c * 512 + 2 * tid] = level(tid & 15);
        lut[c * 512 + 2 * tid + 1] = level(tid >> 4);
      }
    }
    if constexpr (DQ) {
      reinterpret_cast<float*>(smem + kLdsDq)[tid] = ((float)tid / 255.0f) * (*g.scales.scale_of_scales);
      if constexpr (PAIR)
        reinterpret_cast<float*>(smem + kLdsDq + 1024)[tid] = ((float)tid / 255.0f) * (*g.scales2.scale_of_scales);
    }
  }
  const int nk = min(g.k_steps, g.K / kBK - kb);  // K steps of this workgroup (>= 1)

  // Every role passes the same nk + 1 workgroup barriers: the LUTs, steps 0
  // and 1 ready, then one per further step.
  if (wave >= 4) {
    constexpr int kBRing = 4;
    const int d = tid - 256;
    // thread d fills W tile columns 16 (d / 32) .. + 15; in PAIR mode the
    // waves with d < 128 read gate, the others up (each wave one weight)
    const int st = d >> 5;
    const bool second = PAIR && st >= 4;
    const BSrc src{second ? g.packed2 : g.packed, second ? g.scales2 : g.scales,
                   TRANS ? n0 : n0 + 16 * (PAIR ? st & 3 : st)};
    const int dqt = second ? 1 : 0;
    auto ld = [&](BStep& B, int k0) {
      if constexpr (TRANS) load_bt<DQ>(B, g, src, k0, d);
      else load_b<DQ, STRIPED>(B, g, src, k0, d);
    };
    auto st_b = [&](const BStep& B, int buf) {
      if constexpr (TRANS) store_bt<DQ>(B, smem, buf, d);
      else store_b<DQ, STRIPED>(B, smem, buf, d, dqt);
    };
    BStep Br[kBRing];
#pragma unroll
    for (int r = 0; r < kBRing; ++r) ld(Br[r], kbase + min(r, nk - 1) * kBK);
    lds_barrier();  // LUTs visible
    st_b(Br[0], 0);
    ld(Br[0], kbase + min(kBRing, nk - 1) * kBK);
    if (nk > 1) {
      st_b(Br[1], 1);
      ld(Br[1], kbase + min(kBRing + 1, nk - 1) * kBK);
    }
    lds_barrier();  // steps 0 and 1 ready
    // step t2 (from 2 on) into W buffer t2 % 3 from ring slot t2 % kBRing,
    // then the barrier that publishes it
    auto produce = [&](int t2, int slot) {
      st_b(Br[slot], t2 % kBStages);
      ld(Br[slot], kbase + min(t2 + kBRing, nk - 1) * kBK);
      lds_barrier();
    };
    int t2 = 2;
    for (; t2 + kBRing <= nk; t2 += kBRing) {
#pragma unroll
      for (int u = 0; u < kBRing; ++u) produce(t2 + u, (2 + u) % kBRing);
    }
    // the last (at most 3) steps straight-line: in a loop the compiler's
    // wait for the ring slot's codes degrades to vmcnt(0), which also waits
    // for the loads issued one step earlier
    if (t2 < nk) {
      produce(t2++, 2);
      if (t2 < nk) {
        produce(t2++, 3);
        if (t2 < nk) produce(t2++, 0);
      }
    }
    if (nk >= 2) lds_barrier();  // the last step's barrier: nothing left to produce
    UNIFUR_WAIT_VMCNT(0);        // drain the clamped reloads before the wave exits
    return;
  }

  // rows past M read as zero (buffer bound)
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(g.x), (short)0, (int)((uint32_t)g.M * (uint32_t)g.K * 2u), 0x00020000);
  const int awave = kLdsA + w4 * (kATileBytes / 4);
  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  load_a(xr, g.K, row0, kbase, awave, lane);
  if (nk > 1) load_a(xr, g.K, row0, kbase + kBK, awave + kATileBytes, lane);
  lds_barrier();  // LUTs visible
  lds_barrier();  // steps 0 and 1 ready
  if (nk > 1) UNIFUR_WAIT_VMCNT(8);  // this wave's X copies of step 0 landed
  else UNIFUR_WAIT_VMCNT(0);
  Frags Fa, Fb;
  read_frags(Fa, awave, kLdsB, 0, lane);
  int sa = 0, sb = 0;  // X stage and W buffer of step s
  // One K step; COPY2: copy step s + 2's X, NEXT: read step s + 1's first
  // slice at the end.  The main loop takes both, the last two steps are
  // peeled, so that the LDS wait counts stay exact (no branch merges them).
  auto step = [&](int s, auto copy2, auto next) {
    constexpr bool kCopy2 = decltype(copy2)::value, kNext = decltype(next)::value;
    const int ab = awave + sa * kATileBytes, bb = kLdsB + sb * kBTileBytes;
    const int sa1 = sa == 2 ? 0 : sa + 1, sb1 = sb == kBStages - 1 ? 0 : sb + 1;
    // the first slice's fragments were read during the previous step (and
    // waited for by its barrier): nothing is in flight on LDS here
    __builtin_amdgcn_s_waitcnt(0xc07f);
    // step s + 2 goes to the stage step s - 1 used: all its reads completed
    // before that step's last MFMAs issued
    if constexpr (kCopy2)
      load_a(xr, g.K, row0, kbase + (s + 2) * kBK, awave + (sa == 0 ? 2 : sa - 1) * kATileBytes, lane);
    read_frags(Fb, ab, bb, 1, lane);
    mma_frags(acc, Fa);
    read_frags(Fa, ab, bb, 2, lane);
    mma_frags(acc, Fb);
    read_frags(Fb, ab, bb, 3, lane);
    mma_frags(acc, Fa);
    if constexpr (kNext) {
      // step s + 1's W tile was published by the previous barrier; its X
      // copies are the older of the (up to) two groups in flight
      if constexpr (kCopy2) UNIFUR_WAIT_VMCNT(8);
      else UNIFUR_WAIT_VMCNT(0);
      read_frags(Fa, awave + sa1 * kATileBytes, kLdsB + sb1 * kBTileBytes, 0, lane);
    }
    mma_frags(acc, Fb);
    if constexpr (kNext) lds_barrier();
    sa = sa1;
    sb = sb1;
  };
  using yes = std::true_type;
  using no = std::false_type;
  int s = 0;
  for (; s + 2 < nk; ++s) step(s, yes{}, yes{});
  if (s + 1 < nk) step(s++, no{}, yes{});
  step(s, no{}, no{});

  finish_tile<YBF16, LORA, PAIR>(g, acc, yout, row0, n0, lane, (uint32_t)awave, (uint32_t)(awave + kATileBytes));
}

template <bool DQ, bool YBF16, bool LORA, bool STRIPED, bool PAIR = false, bool TRANS = false>
hipError_t launch_g(const GemmArgs& g, hipStream_t stream) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  const void* fn = reinterpret_cast<const void*>(&gemm_kernel<DQ, YBF16, LORA, STRIPED, PAIR, TRANS>);
  if (!(done.load(std::memory_order_acquire) & bit)) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmSmem);
    if (e != hipSuccess) return e;
    done.fetch_or(bit, std::memory_order_acq_rel);
  }
  const int tiles = g.tile_count ? g.tile_count : ((g.M + kBM - 1) / kBM) * g.tiles_n;
  gemm_kernel<DQ, YBF16, LORA, STRIPED, PAIR, TRANS><<<tiles * g.k_splits, kGemmThreads, kGemmSmem, stream>>>(g);
  return hipGetLastError();
}

// ------------------------------------------------------------ LoRA x A ------
// The adapter operands of the fused epilogue, in bf16 layouts whose MFMA
// fragments are single 16-byte loads (pad = rank rounded up to 16, zero past
// the rank):
//   * lora_prep_kernel: at[pad][K] = A transposed and bt[N][pad] = B
//     transposed, one element of at or bf16 pair of bt per thread (at
//     config 3 its ~4.8 us are mostly the launch itself);
//   * lora_xa_kernel: xa[M][pad] = bf16(scaling * (X A)) -- the first factor
//     of LoraAdapter::forward (src/quantize.rs:619-624) with the scaling
//     folded in -- R rows x 16 columns per workgroup (R = 16, or 8 or 4 when
//     16-row workgroups would not cover the CUs: the MFMA's other rows read
//     zero); eight waves split K (v_mfma_f32_16x16x32_bf16, X and at straight
//     from memory, eight steps of 16-byte loads in flight) and add their
//     slices through LDS in wave order.

// The two factors are read through strides: element (k, j) of the first
// at a[k sak + j saj], element (j, n) of the second at b[j sbj + n sbn]
// (A [K][r] and B [r][N] as stored for the forward; B read as B^T and A as
// A^T for dX = dY W^T, whose adapter term is ((dY scaling) B^T) A^T).
__global__ __launch_bounds__(256) void lora_prep_kernel(const float* __restrict__ a, size_t sak, size_t saj,
                                                        const float* __restrict__ b, size_t sbj, size_t sbn, int K,
                                                        int N, int rank, int pad, uint16_t* __restrict__ at,
                                                        uint32_t* __restrict__ bt2) {
  // one thread per element of at [pad][K] (consecutive threads: consecutive
  // k, so the stores coalesce), then one per bf16 pair of bt [N][pad]
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t n_at = (size_t)pad * K;
  if (t < n_at) {
    const int j = (int)(t / (size_t)K), k = (int)(t - (size_t)j * K);
    at[t] = j < rank ? (uint16_t)(pack_bf16x2(a[(size_t)k * sak + (size_t)j * saj], 0.0f) & 0xffffu) : 0;
  } else if (t < n_at + (size_t)N * pad / 2) {
    const size_t u = t - n_at;  // bt element pair (n, 2 jp), (n, 2 jp + 1)
    const int half = pad / 2;
    const int n = (int)(u / (size_t)half), r0 = 2 * (int)(u - (size_t)n * half), r1 = r0 + 1;
    bt2[u] = pack_bf16x2(r0 < rank ? b[(size_t)r0 * sbj + (size_t)n * sbn] : 0.0f,
                         r1 < rank ? b[(size_t)r1 * sbj + (size_t)n * sbn] : 0.0f);
  }
}

constexpr int kXaWaves = 8;
constexpr int kXaBatch = 8;  // k32 steps whose loads are in flight together

template <int R>
__global__ __launch_bounds__(64 * kXaWaves) void lora_xa_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ at, int M, int K,
                                                                int pad, float scaling, uint16_t* __restrict__ xa) {
  __shared__ float red[kXaWaves][256];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m0 = blockIdx.x * R, c0 = blockIdx.y * 16;
  const int kq = K / kXaWaves;  // a multiple of 8 (K % 64 == 0)
  const int kbeg = wv * kq, kend = kbeg + kq;
  // rows past M read as zero (buffer bound), and so does a step past the
  // wave's slice (an offset past the end): no load sits behind a branch
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(at), (short)0, (int)((uint32_t)pad * (uint32_t)K * 2u), 0x00020000);
  const bool row_ok = (lane & 15) < R;  // rows past the tile's R read zero
  const uint32_t xrow = (uint32_t)(m0 + (lane & 15)) * (uint32_t)K * 2u;
  const uint32_t arow = (uint32_t)(c0 + (lane & 15)) * (uint32_t)K * 2u;
  const int kl = 8 * (lane >> 4);  // this lane's 8 k of each 32
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = kbeg; k0 < kend; k0 += 32 * kXaBatch) {
    bf16x8 xv[kXaBatch], av[kXaBatch];
#pragma unroll
    for (int q = 0; q < kXaBatch; ++q) {
      const int k = k0 + 32 * q + kl;
      const bool ok = k < kend;  // K / 8 may end inside a 32-k step: mask per 8-k group
      xv[q] = __builtin_bit_cast(
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xr, ok && row_ok ? xrow + (uint32_t)k * 2u : 0xffffffffu, 0, 0));
      av[q] = __builtin_bit_cast(
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(ar, ok ? arow + (uint32_t)k * 2u : 0xffffffffu, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);  // the whole batch's loads are in flight before the first MFMA
#pragma unroll
    for (int q = 0; q < kXaBatch; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xv[q], av[q], acc, 0, 0, 0);
  }
  // acc[e] = C[row 4 (lane / 16) + e][col lane % 16]; add the K slices in order
#pragma unroll
  for (int e = 0; e < 4; ++e) red[wv][(4 * (lane >> 4) + e) * 16 + (lane & 15)] = acc[e];
  __syncthreads();
  const int t = threadIdx.x;
  if (t < 16 * R) {
    const int m = m0 + t / 16;
    if (m < M) {
      float v = red[0][t];
#pragma unroll
      for (int w = 1; w < kXaWaves; ++w) v += red[w][t];
      xa[(size_t)m * pad + c0 + (t & 15)] = (uint16_t)(pack_bf16x2(v * scaling, 0.0f) & 0xffffu);
    }
  }
}

}  // namespace

bool gemm_supported(int M, int K, int N, const void* x) {
  // every X offset a workgroup forms, rows past M included, stays below 2^31
  return M > 0 && K >= kBK && K % kBK == 0 && N % kBN == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
         ((uint64_t)M + kBM) * (uint64_t)K * 2u < (1ull << 31);
}

int lora_pad(int rank) { return (rank + 15) / 16 * 16; }

namespace {

hipError_t lora_operands(const uint16_t* x, const float* a, size_t sak, size_t saj, const float* b, size_t sbj,
                         size_t sbn, int M, int K, int N, int rank, float scaling, uint16_t* at, uint16_t* bt,
                         uint16_t* xa, hipStream_t stream) {
  if (rank < 1 || rank > 64 || K % 64 != 0) return hipErrorInvalidValue;
  const int pad = lora_pad(rank);
  const size_t prep = (size_t)pad * K + (size_t)N * pad / 2;
  lora_prep_kernel<<<(unsigned)((prep + 255) / 256), 256, 0, stream>>>(a, sak, saj, b, sbj, sbn, K, N, rank, pad, at,
                                                                       reinterpret_cast<uint32_t*>(bt));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // rows per workgroup: 16 while that covers the CUs, else 8 or 4
  const dim3 block(64 * kXaWaves);
  const unsigned cols = (unsigned)(pad / 16);
  if ((long)((M + 15) / 16) * cols >= 256)
    lora_xa_kernel<16><<<dim3((unsigned)((M + 15) / 16), cols), block, 0, stream>>>(x, at, M, K, pad, scaling, xa);
  else if ((long)((M + 7) / 8) * cols >= 256)
    lora_xa_kernel<8><<<dim3((unsigned)((M + 7) / 8), cols), block, 0, stream>>>(x, at, M, K, pad, scaling, xa);
  else
    lora_xa_kernel<4><<<dim3((unsigned)((M + 3) / 4), cols), block, 0, stream>>>(x, at, M, K, pad, scaling, xa);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_lora_operands(const uint16_t* x, const float* a, const float* b, int M, int K, int N, int rank,
                                float scaling, uint16_t* at, uint16_t* bt, uint16_t* xa, hipStream_t stream) {
  return lora_operands(x, a, (size_t)rank, 1, b, (size_t)N, 1, M, K, N, rank, scaling, at, bt, xa, stream);
}

hipError_t launch_lora_operands_dx(const uint16_t* dy, const float* a, const float* b, int M, int d_in, int d_out,
                                   int rank, float scaling, uint16_t* at, uint16_t* bt, uint16_t* xa,
                                   hipStream_t stream) {
  // first factor B^T [d_out][r] (B [r][d_out] read by columns), second A^T
  // [r][d_in] (A [d_in][r] read by columns); K = d_out, N = d_in
  return lora_operands(dy, b, 1, (size_t)d_out, a, 1, (size_t)rank, M, d_out, d_in, rank, scaling, at, bt, xa, stream);
}

namespace {

// Split-K reduction: y[m][n] = sum over the splits, in split order, of
// partials[s][m][n] (+ bias[n]), four consecutive outputs per thread.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partials, int splits,
                                                            size_t mn4, int n4, const float* __restrict__ bias,
                                                            void* __restrict__ y, int y_bf16) {
  const size_t stride = mn4;  // f32x4 per split
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn4; i += (size_t)gridDim.x * blockDim.x) {
    f32x4 v = reinterpret_cast<const f32x4*>(partials)[i];
    for (int q = 1; q < splits; ++q) {
      const f32x4 w = reinterpret_cast<const f32x4*>(partials)[i + q * stride];
      v = f32x4{v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w};
    }
    if (bias) {
      const f32x4 b4 = reinterpret_cast<const f32x4*>(bias)[i % (size_t)n4];
      v = f32x4{v.x + b4.x, v.y + b4.y, v.z + b4.z, v.w + b4.w};
    }
    if (y_bf16)
      reinterpret_cast<u32x2*>(y)[i] = u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
    else
      reinterpret_cast<f32x4*>(y)[i] = v;
  }
}

// The SwiGLU pair's reduction: gate and up each summed over the splits in
// split order from partials[s][m][2 N] (gate columns, then up), then
// h[m][n] = bf16(silu(gate) * up), four outputs per thread.
__global__ __launch_bounds__(256) void splitk_silu_reduce_kernel(const float* __restrict__ partials, int splits,
                                                                 size_t split_stride, uint32_t n4_row, size_t mn4,
                                                                 uint16_t* __restrict__ h) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn4; i += (size_t)gridDim.x * blockDim.x) {
    const size_t m = i / n4_row, c4 = i - m * n4_row;
    const float* gp = partials + m * 8 * n4_row + c4 * 4;  // row m: 2 N floats
    f32x4 gv = *reinterpret_cast<const f32x4*>(gp);
    f32x4 uv = *reinterpret_cast<const f32x4*>(gp + 4 * n4_row);
    for (int q = 1; q < splits; ++q) {
      const f32x4 g2 = *reinterpret_cast<const f32x4*>(gp + q * split_stride);
      const f32x4 u2 = *reinterpret_cast<const f32x4*>(gp + q * split_stride + 4 * n4_row);
      gv = f32x4{gv.x + g2.x, gv.y + g2.y, gv.z + g2.z, gv.w + g2.w};
      uv = f32x4{uv.x + u2.x, uv.y + u2.y, uv.z + u2.z, uv.w + u2.w};
    }
    reinterpret_cast<u32x2*>(h)[i] = u32x2{pack_bf16x2(silu_times(gv.x, uv.x), silu_times(gv.y, uv.y)),
                                          pack_bf16x2(silu_times(gv.z, uv.z), silu_times(gv.w, uv.w))};
  }
}

// The split-K reduction of only the tiles [t0, t0 + gridDim.x / 8) of a
// launch (its other tiles were computed whole): 8 workgroups per tile, 32 of
// its rows each, four outputs per thread, the splits added in order; PAIR:
// gate and up summed, then bf16 silu(gate) * up into h.
template <bool PAIR>
__global__ __launch_bounds__(256) void splitk_reduce_tiles_kernel(const float* __restrict__ partials, int splits,
                                                                  size_t split_stride, int M, int N, int tiles_n,
                                                                  int t0, const float* __restrict__ bias,
                                                                  void* __restrict__ y, int y_bf16) {
  constexpr int kCols = PAIR ? kBN / 2 : kBN, kC4 = kCols / 4;
  const int t = t0 + (int)blockIdx.x / 8;
  const int m0 = (t / tiles_n) * kBM + ((int)blockIdx.x % 8) * 32, n0 = (t % tiles_n) * kCols;
  const size_t ldp = PAIR ? 2 * (size_t)N : (size_t)N;  // a partial row: gate columns, then up
  for (int i = threadIdx.x; i < 32 * kC4; i += 256) {
    const int m = m0 + i / kC4, n = n0 + 4 * (i % kC4);
    if (m >= M) continue;
    const float* p = partials + (size_t)m * ldp + n;
    f32x4 v = *reinterpret_cast<const f32x4*>(p);
    f32x4 u = PAIR ? *reinterpret_cast<const f32x4*>(p + N) : f32x4{};
    for (int q = 1; q < splits; ++q) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(p + q * split_stride);
      v = f32x4{v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w};
      if constexpr (PAIR) {
        const f32x4 w2 = *reinterpret_cast<const f32x4*>(p + q * split_stride + N);
        u = f32x4{u.x + w2.x, u.y + w2.y, u.z + w2.z, u.w + w2.w};
      }
    }
    const size_t o = (size_t)m * N + n;
    if constexpr (PAIR) {
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(y) + o) =
          u32x2{pack_bf16x2(silu_times(v.x, u.x), silu_times(v.y, u.y)),
                pack_bf16x2(silu_times(v.z, u.z), silu_times(v.w, u.w))};
    } else {
      if (bias) {
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(bias + n);
        v = f32x4{v.x + b4.x, v.y + b4.y, v.z + b4.z, v.w + b4.w};
      }
      if (y_bf16)
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(y) + o) = u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
      else
        *reinterpret_cast<f32x4*>(static_cast<float*>(y) + o) = v;
    }
  }
}

}  // namespace

int gemm_tail_splits(int M, int K, int N, bool pair) {
  // a grid of more than one round whose last round is at most half full:
  // the whole rounds' tiles run whole and the last round's tiles split d_in
  // (f32 partials, an ordered reduction of those tiles), so that the last
  // round fills the CUs instead of leaving most of them idle
  const long tiles = (long)((M + kBM - 1) / kBM) * (pair ? N / (kBN / 2) : N / kBN);
  const long rem = tiles % 256;
  if (tiles <= 256 || rem == 0 || gemm_k_splits(M, K, N, pair) > 1) return 1;
  const int steps = K / kBK;
  int splits = 1;
  while (rem * splits * 2 <= 256 && steps / (splits * 2) >= 16) splits *= 2;
  return splits;
}

int gemm_k_splits(int M, int K, int N, bool pair) {
  // grids of fewer than ~200 tiles leave CUs idle (one 148 KiB workgroup per
  // CU): split d_in so the grid reaches ~256 workgroups, each over at least
  // 16 K steps.  A grid of more than one round stays whole: with every CU
  // busy the part runs at its power limit, and splitting the 344 tiles of
  // the 7B-shaped gate/up pair at 512 rows two ways measured 134 us plus a
  // 16 us reduction against 137 us whole.
  const long tiles = (long)((M + kBM - 1) / kBM) * (pair ? N / (kBN / 2) : N / kBN);
  const int steps = K / kBK;
  int splits = 1;
  while (tiles * splits * 2 <= 256 && steps / (splits * 2) >= 16) splits *= 2;
  return splits;
}

namespace {

GemmArgs gemm_args(const uint16_t* x, const uint8_t* packed, const ScalesArg& scales, int M, int K, int N, void* y,
                   bool y_bf16, int k_splits, float* partials) {
  GemmArgs g{};
  g.x = x;
  g.packed = packed;
  g.scales = scales;
  g.M = M;
  g.K = K;
  g.N = N;
  g.y = y;
  g.y_bf16 = y_bf16;
  g.y_aligned = (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
  g.tiles_n = N / kBN;
  g.ldy = N;
  const int steps = K / kBK;
  g.k_splits = k_splits;
  g.k_steps = (steps + k_splits - 1) / k_splits;
  g.partials = partials;
  return g;
}

// every split of k_splits has a K step
bool splits_ok(int K, int k_splits) {
  const int steps = K / kBK;
  return k_splits >= 1 && (k_splits == 1 || ((steps + k_splits - 1) / k_splits) * (k_splits - 1) < steps);
}

unsigned reduce_blocks(size_t n4) { return (unsigned)std::min<size_t>((n4 + 255) / 256, 4096); }

}  // namespace

hipError_t launch_gemm(const uint16_t* x, const uint8_t* packed, const ScalesArg& scales, int M, int K, int N,
                       const float* bias, const uint16_t* lora_xa, const uint16_t* lora_bt, int lora_rank, void* y,
                       bool y_bf16, bool striped, hipStream_t stream, int k_splits, float* partials, int tail_splits) {
  if (!splits_ok(K, k_splits) || (k_splits > 1 && (!partials || lora_xa || (reinterpret_cast<uintptr_t>(y) & 15u) != 0)))
    return hipErrorInvalidValue;
  GemmArgs g = gemm_args(x, packed, scales, M, K, N, y, y_bf16, k_splits, partials);
  g.bias = bias;
  g.lora_xa = lora_xa;
  g.lora_bt = lora_bt;
  g.lora_rank = lora_rank;
  g.lora_pad = lora_pad(lora_rank);
  if (k_splits > 1) {
    // raw f32 sums into the partials, then the ordered reduction
    g.bias = nullptr;
    g.y_bf16 = 0;
    g.y_aligned = 1;
    const bool dq0 = scales.kind == kScalesDQ;
    hipError_t e = dq0 ? (striped ? launch_g<true, false, false, true>(g, stream) : launch_g<true, false, false, false>(g, stream))
                       : (striped ? launch_g<false, false, false, true>(g, stream) : launch_g<false, false, false, false>(g, stream));
    if (e != hipSuccess) return e;
    const size_t mn4 = (size_t)M * N / 4;
    splitk_reduce_kernel<<<reduce_blocks(mn4), 256, 0, stream>>>(partials, k_splits, mn4, N / 4, bias, y, y_bf16);
    return hipGetLastError();
  }
  const bool dq = scales.kind == kScalesDQ;
  const bool lora = lora_xa != nullptr;
  if (tail_splits > 1) {
    if (lora || !partials || (reinterpret_cast<uintptr_t>(y) & 15u) != 0 || !splits_ok(K, tail_splits))
      return hipErrorInvalidValue;
    // the whole rounds' tiles, then the last round's split (see gemm_tail_splits)
    const int tiles = ((M + kBM - 1) / kBM) * g.tiles_n, whole = tiles - tiles % 256;
    g.tile_count = whole;
    hipError_t e = dq ? (y_bf16 ? (striped ? launch_g<true, true, false, true>(g, stream) : launch_g<true, true, false, false>(g, stream))
                                : (striped ? launch_g<true, false, false, true>(g, stream) : launch_g<true, false, false, false>(g, stream)))
                      : (y_bf16 ? (striped ? launch_g<false, true, false, true>(g, stream) : launch_g<false, true, false, false>(g, stream))
                                : (striped ? launch_g<false, false, false, true>(g, stream) : launch_g<false, false, false, false>(g, stream)));
    if (e != hipSuccess) return e;
    GemmArgs t = gemm_args(x, packed, scales, M, K, N, partials, false, tail_splits, partials);
    t.y_aligned = 1;
    t.tile_begin = whole;
    t.tile_count = tiles - whole;
    e = dq ? (striped ? launch_g<true, false, false, true>(t, stream) : launch_g<true, false, false, false>(t, stream))
           : (striped ? launch_g<false, false, false, true>(t, stream) : launch_g<false, false, false, false>(t, stream));
    if (e != hipSuccess) return e;
    splitk_reduce_tiles_kernel<false><<<(tiles - whole) * 8, 256, 0, stream>>>(
        partials, tail_splits, (size_t)M * N, M, N, g.tiles_n, whole, bias, y, y_bf16);
    return hipGetLastError();
  }
#define UNIFUR_GEMM_CASE(D, B, R)                                                     \
  if (dq == D && y_bf16 == B && lora == R)                                          \
    return striped ? launch_g<D, B, R, true>(g, stream) : launch_g<D, B, R, false>(g, stream);
  UNIFUR_GEMM_CASE(true, true, true)
  UNIFUR_GEMM_CASE(true, true, false)
  UNIFUR_GEMM_CASE(true, false, true)
  UNIFUR_GEMM_CASE(true, false, false)
  UNIFUR_GEMM_CASE(false, true, true)
  UNIFUR_GEMM_CASE(false, true, false)
  UNIFUR_GEMM_CASE(false, false, true)
  UNIFUR_GEMM_CASE(false, false, false)
#undef UNIFUR_GEMM_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_pair(const uint16_t* x, const uint8_t* gate_packed, const ScalesArg& gate_scales,
                            const uint8_t* up_packed, const ScalesArg& up_scales, int M, int K, int N, uint16_t* h,
                            bool striped, hipStream_t stream, int k_splits, float* partials, int tail_splits) {
  if (gate_scales.kind != up_scales.kind || N % 64 != 0 || !splits_ok(K, k_splits) ||
      (k_splits > 1 && !partials))
    return hipErrorInvalidValue;
  GemmArgs g = gemm_args(x, gate_packed, gate_scales, M, K, N, h, true, k_splits, partials);
  g.packed2 = up_packed;
  g.scales2 = up_scales;
  g.tiles_n = N / (kBN / 2);
  const bool dq = gate_scales.kind == kScalesDQ;
  if (k_splits == 1 && tail_splits > 1) {
    if (!partials || !splits_ok(K, tail_splits)) return hipErrorInvalidValue;
    // the whole rounds' tiles store silu(g) * u; the last round's tiles
    // split d_in (see gemm_tail_splits)
    const int tiles = ((M + kBM - 1) / kBM) * g.tiles_n, whole = tiles - tiles % 256;
    g.tile_count = whole;
    hipError_t e = dq ? (striped ? launch_g<true, true, false, true, true>(g, stream) : launch_g<true, true, false, false, true>(g, stream))
                      : (striped ? launch_g<false, true, false, true, true>(g, stream) : launch_g<false, true, false, false, true>(g, stream));
    if (e != hipSuccess) return e;
    GemmArgs t = gemm_args(x, gate_packed, gate_scales, M, K, N, partials, false, tail_splits, partials);
    t.packed2 = up_packed;
    t.scales2 = up_scales;
    t.tiles_n = g.tiles_n;
    t.y_aligned = 1;
    t.ldy = 2 * N;
    t.tile_begin = whole;
    t.tile_count = tiles - whole;
    e = dq ? (striped ? launch_g<true, false, false, true, true>(t, stream) : launch_g<true, false, false, false, true>(t, stream))
           : (striped ? launch_g<false, false, false, true, true>(t, stream) : launch_g<false, false, false, false, true>(t, stream));
    if (e != hipSuccess) return e;
    splitk_reduce_tiles_kernel<true><<<(tiles - whole) * 8, 256, 0, stream>>>(
        partials, tail_splits, (size_t)M * 2 * N, M, N, g.tiles_n, whole, nullptr, h, 1);
    return hipGetLastError();
  }
  if (k_splits == 1) {
    return dq ? (striped ? launch_g<true, true, false, true, true>(g, stream) : launch_g<true, true, false, false, true>(g, stream))
              : (striped ? launch_g<false, true, false, true, true>(g, stream) : launch_g<false, true, false, false, true>(g, stream));
  }
  // raw gate and up sums into partials[s][M][2 N], then the ordered
  // reduction with silu(gate) * up
  g.y_bf16 = 0;
  g.y_aligned = 1;
  g.ldy = 2 * N;
  hipError_t e = dq ? (striped ? launch_g<true, false, false, true, true>(g, stream) : launch_g<true, false, false, false, true>(g, stream))
                    : (striped ? launch_g<false, false, false, true, true>(g, stream) : launch_g<false, false, false, false, true>(g, stream));
  if (e != hipSuccess) return e;
  const size_t mn4 = (size_t)M * N / 4;
  splitk_silu_reduce_kernel<<<reduce_blocks(mn4), 256, 0, stream>>>(partials, k_splits, (size_t)M * 2 * N,
                                                                     (uint32_t)(N / 4), mn4, h);
  return hipGetLastError();
}

hipError_t launch_gemm_dx(const uint16_t* dy, const uint8_t* packed, const ScalesArg& scales, int M, int d_in, int d_out,
                          const uint16_t* lora_xa, const uint16_t* lora_bt, int lora_rank, void* dx, bool dx_bf16,
                          hipStream_t stream, int k_splits, float* partials) {
  // outputs d_in (128-column tiles of W rows), reduction d_out (64-column blocks of W)
  if (!splits_ok(d_out, k_splits) || d_in % kBN != 0 ||
      (k_splits > 1 && (!partials || lora_xa || (reinterpret_cast<uintptr_t>(dx) & 15u) != 0)))
    return hipErrorInvalidValue;
  GemmArgs g = gemm_args(dy, packed, scales, M, d_out, d_in, dx, dx_bf16, k_splits, partials);
  g.lora_xa = lora_xa;
  g.lora_bt = lora_bt;
  g.lora_rank = lora_rank;
  g.lora_pad = lora_pad(lora_rank);
  const bool dq = scales.kind == kScalesDQ;
  if (k_splits > 1) {
    g.y_bf16 = 0;
    g.y_aligned = 1;
    hipError_t e = dq ? launch_g<true, false, false, true, false, true>(g, stream)
                      : launch_g<false, false, false, true, false, true>(g, stream);
    if (e != hipSuccess) return e;
    const size_t mn4 = (size_t)M * d_in / 4;
    splitk_reduce_kernel<<<reduce_blocks(mn4), 256, 0, stream>>>(partials, k_splits, mn4, d_in / 4, nullptr, dx,
                                                                 dx_bf16);
    return hipGetLastError();
  }
  const bool lora = lora_xa != nullptr;
#define UNIFUR_GEMM_DX_CASE(D, B, R) \
  if (dq == D && dx_bf16 == B && lora == R) return launch_g<D, B, R, true, false, true>(g, stream);
  UNIFUR_GEMM_DX_CASE(true, true, true)
  UNIFUR_GEMM_DX_CASE(true, true, false)
  UNIFUR_GEMM_DX_CASE(true, false, true)
  UNIFUR_GEMM_DX_CASE(true, false, false)
  UNIFUR_GEMM_DX_CASE(false, true, true)
  UNIFUR_GEMM_DX_CASE(false, true, false)
  UNIFUR_GEMM_DX_CASE(false, false, true)
  UNIFUR_GEMM_DX_CASE(false, false, false)
#undef UNIFUR_GEMM_DX_CASE
  return hipErrorInvalidValue;
}

}  // namespace unifur
