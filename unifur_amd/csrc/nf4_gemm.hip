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
// Tiling.  A 256-thread workgroup (4 waves, 2 x 2) computes a 128 x 128
// output tile; each wave owns 64 x 64 (2 x 2 MFMA 32x32x16 tiles, f32
// accumulators).  K advances in steps of 64 through double-buffered LDS:
// while the MFMAs consume step k, the global loads of step k + 1 (X rows and
// NF4 codes + scales) are in flight; afterwards the X tile is written to LDS
// and the codes are expanded (byte LUT -> level pair, x block scale, -> bf16)
// into the B tile, stored [n][k] so that each MFMA operand fetch is one
// 16-byte ds_read.  Both tiles use a 16-byte-chunk XOR swizzle,
// chunk ^ ((row % 8) ^ (row / 8 % 8)), which makes the operand reads (8
// consecutive rows, one chunk) and the tile writes conflict-free.
#include "nf4_gemm.hpp"

#include <atomic>

namespace unifur {
namespace {

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kGemmThreads = 256;
constexpr int kTileBytes = kBM * kBK * 2;               // one bf16 tile (A or B): 16 KiB
constexpr int kLdsA = 0;                                // 2 buffers
constexpr int kLdsB = 2 * kTileBytes;                   // 2 buffers
constexpr int kLdsLut = 4 * kTileBytes;                 // byte LUT, 256 x f32x2
constexpr int kLdsDq = kLdsLut + 256 * 8;               // DQ scale LUT, 256 x f32
constexpr size_t kGemmSmem = kLdsDq + 256 * 4;          // 67 KiB: two workgroups per CU

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) const f32x2 lds_f32x2_c;

struct GemmArgs {
  const uint16_t* x;  // [M, K] bf16
  const uint8_t* packed;
  ScalesArg scales;
  int M, K, N;
  const float* bias;     // [N] or null
  const float* lora_xa;  // [M, lora_pad]: scaling * (x A), zero past lora_rank; or null
  const float* lora_b;   // [lora_rank, N]
  int lora_rank, lora_pad;
  void* y;  // [M, N] f32 or bf16
  int y_bf16;
  int tiles_n;  // N / kBN
};

// 16-byte chunk swizzle of a 128-byte tile row (8 chunks).
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row & 7) ^ ((row >> 3) & 7)); }

__device__ __forceinline__ uint32_t lds_addr(int base, int row, int chunk) {
  return (uint32_t)(base + row * (kBK * 2) + swz(row, chunk) * 16);
}

// Global-memory operands of one K step, held in registers between the loads
// and the LDS writes.
template <bool DQ>
struct StepLoads {
  u32x4 a[4];        // X: rows t/8 + 32 p, 16-byte chunk t % 8
  uint32_t code[4];  // W: rows 4 (t / 16) + i, bytes of columns 8 (t % 16) .. + 7
  uint32_t scale[4];
};

template <bool DQ>
__device__ __forceinline__ void load_step(StepLoads<DQ>& L, const GemmArgs& g, int m0, int n0, int k0, int tid) {
  // X tile: 128 rows x 64 k; rows past M read as zero (buffer bound).
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(g.x), (short)0, (int)((uint32_t)g.M * (uint32_t)g.K * 2u), 0x00020000);
  const int ar = tid >> 3, ach = tid & 7;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t off = ((uint32_t)(m0 + ar + 32 * p) * (uint32_t)g.K + (uint32_t)(k0 + ach * 8)) * 2u;
    L.a[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
  }
  // W codes: 64 rows x 128 columns = 64 bytes per row.
  const int c = tid & 15, g4 = tid >> 4;
  const uint32_t row_bytes = (uint32_t)g.N / 2;
  const uint32_t bpr = (uint32_t)g.N / kBlock;
  const uint8_t* cp = g.packed + (size_t)(k0 + 4 * g4) * row_bytes + (n0 + 8 * c) / 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) L.code[i] = *reinterpret_cast<const uint32_t*>(cp + (size_t)i * row_bytes);
  const size_t blk = (size_t)(k0 + 4 * g4) * bpr + (n0 + 8 * c) / kBlock;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DQ)
      L.scale[i] = g.scales.dq_codes[blk + (size_t)i * bpr];
    else
      L.scale[i] = __float_as_uint(g.scales.absmax[blk + (size_t)i * bpr]);
  }
}

// X registers -> LDS A tile; codes -> dequantized bf16 B tile [n][k].
template <bool DQ>
__device__ __forceinline__ void store_step(const StepLoads<DQ>& L, unsigned char* smem, int buf, int tid) {
  const int ar = tid >> 3, ach = tid & 7;
#pragma unroll
  for (int p = 0; p < 4; ++p)
    *reinterpret_cast<lds_u32x4*>((size_t)lds_addr(kLdsA + buf * kTileBytes, ar + 32 * p, ach)) = L.a[p];

  const int c = tid & 15, g4 = tid >> 4;
  const float* dq_lut = reinterpret_cast<const float*>(smem + kLdsDq);
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = DQ ? dq_lut[L.scale[i] & 0xffu] : __uint_as_float(L.scale[i]);
  // v[i][j]: row k0 + 4 g4 + i, column n0 + 8 c + j; value level[code] * scale
  // (one f32 multiply, as the reference's dequantize), then bf16.
  float v[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (L.code[i] >> (8 * b)) & 0xffu;
      const f32x2 lv = *reinterpret_cast<lds_f32x2_c*>((size_t)(kLdsLut + byte * 8));
      v[i][2 * b] = lv.x * s[i];
      v[i][2 * b + 1] = lv.y * s[i];
    }
  }
  // column n0 + 8c + j gets k = 4 g4 .. 4 g4 + 3: half (g4 & 1) of chunk g4 / 2
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int n = 8 * c + j;
    const u32x2 w = {pack_bf16x2(v[0][j], v[1][j]), pack_bf16x2(v[2][j], v[3][j])};
    const uint32_t addr = lds_addr(kLdsB + buf * kTileBytes, n, g4 >> 1) + (uint32_t)(g4 & 1) * 8u;
    *reinterpret_cast<lds_u32x2*>((size_t)addr) = w;
  }
}

__device__ __forceinline__ bf16x8 read_frag(int base, int row, int chunk) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<lds_u32x4*>((size_t)lds_addr(base, row, chunk)));
}

template <bool DQ, bool YBF16, bool LORA>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;  // wave's 64 x 64 quadrant

  // XCD-aware tile order: workgroup b runs on XCD b % 8; each XCD gets a
  // contiguous run of tiles in row-major (m, n) order, so the workgroups
  // sharing an X row band sit on the same XCD and share its L2.
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int per_xcd = nb / 8;
  const int t = (nb % 8 == 0) ? (b % 8) * per_xcd + b / 8 : b;
  const int m0 = (t / g.tiles_n) * kBM, n0 = (t % g.tiles_n) * kBN;

  // LUTs: byte -> {level[lo], level[hi]}; DQ code -> scale.
  {
    float* lut = reinterpret_cast<float*>(smem + kLdsLut);
    lut[2 * tid] = level(tid & 15);
    lut[2 * tid + 1] = level(tid >> 4);
    if constexpr (DQ)
      reinterpret_cast<float*>(smem + kLdsDq)[tid] = ((float)tid / 255.0f) * (*g.scales.scale_of_scales);
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int nk = g.K / kBK;
  StepLoads<DQ> L;
  load_step<DQ>(L, g, m0, n0, 0, tid);
  __syncthreads();  // LUTs visible
  store_step<DQ>(L, smem, 0, tid);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_step<DQ>(L, g, m0, n0, (kt + 1) * kBK, tid);
    const int abase = kLdsA + cur * kTileBytes, bbase = kLdsB + cur * kTileBytes;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int ch = kk * 2 + (lane >> 5);
      bf16x8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = read_frag(abase, wr * 64 + i * 32 + (lane & 31), ch);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = read_frag(bbase, wc * 64 + j * 32 + (lane & 31), ch);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_step<DQ>(L, smem, cur ^ 1, tid);
    __syncthreads();
  }

  if constexpr (LORA) {
    // acc += xa[rows, r] . B[r, cols], xa already scaled: one 32x32x16 MFMA
    // per tile and 16 adapter columns (columns past lora_rank contribute zero).
    const int kr = (lane >> 5) * 8;
    for (int r0 = 0; r0 < g.lora_rank; r0 += 16) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int m = m0 + wr * 64 + i * 32 + (lane & 31);
        bf16x8 af;
#pragma unroll
        for (int q = 0; q < 8; ++q)
          af[q] = m < g.M ? (__bf16)g.lora_xa[(size_t)m * g.lora_pad + r0 + kr + q] : (__bf16)0.0f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + wc * 64 + j * 32 + (lane & 31);
          bf16x8 bfr;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int r = r0 + kr + q;
            bfr[q] = r < g.lora_rank ? (__bf16)g.lora_b[(size_t)r * g.N + n] : (__bf16)0.0f;
          }
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bfr, acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // Epilogue: acc[i][j][4 a + e] = C[row 8 a + 4 (lane / 32) + e][col lane % 32].
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wc * 64 + j * 32 + (lane & 31);
      const float bias = g.bias ? g.bias[n] : 0.0f;
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + wr * 64 + i * 32 + 8 * a4 + 4 * (lane >> 5) + e;
          if (m >= g.M) continue;
          const float yv = acc[i][j][4 * a4 + e] + bias;
          const size_t idx = (size_t)m * g.N + n;
          if constexpr (YBF16)
            reinterpret_cast<uint16_t*>(g.y)[idx] = (uint16_t)(pack_bf16x2(yv, 0.0f) & 0xffffu);
          else
            reinterpret_cast<float*>(g.y)[idx] = yv;
        }
      }
    }
  }
}

template <bool DQ, bool YBF16, bool LORA>
hipError_t launch_g(const GemmArgs& g, hipStream_t stream) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  const void* fn = reinterpret_cast<const void*>(&gemm_kernel<DQ, YBF16, LORA>);
  if (!(done.load(std::memory_order_acquire) & bit)) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmSmem);
    if (e != hipSuccess) return e;
    done.fetch_or(bit, std::memory_order_acq_rel);
  }
  const int grid = ((g.M + kBM - 1) / kBM) * g.tiles_n;
  gemm_kernel<DQ, YBF16, LORA><<<grid, kGemmThreads, kGemmSmem, stream>>>(g);
  return hipGetLastError();
}

// ------------------------------------------------------------ LoRA x A ------
// xa[m][j] = scaling * sum_k x[m][k] a[k][j], the first factor of
// LoraAdapter::forward (src/quantize.rs:619-624) with the scaling folded in,
// laid out [M, pad] (pad = rank rounded up to 16, zero past the rank) for the
// fused epilogue.  A workgroup covers 16 rows and 16 adapter columns; its
// four waves take interleaved 32-wide K slices (X rows as the A operand of a
// 16x16x32 MFMA, a as the B operand) and are summed in LDS.
constexpr int kXaWaves = 4;

__global__ __launch_bounds__(64 * kXaWaves) void lora_xa_mfma_kernel(const uint16_t* __restrict__ x,
                                                                    const float* __restrict__ a, int M, int K,
                                                                    int rank, int pad, float scaling,
                                                                    float* __restrict__ xa) {
  __shared__ float part[kXaWaves][16][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int m0 = blockIdx.x * 16, c0 = blockIdx.y * 16;
  const int row = m0 + (lane & 15);
  const int col = c0 + (lane & 15);
  f32x4 acc = {};
#pragma unroll 4
  for (int k = w * 32; k < K; k += 32 * kXaWaves) {
    const int kb = k + (lane >> 4) * 8;
    bf16x8 af, bf;
    if (row < M)
      af = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(x + (size_t)row * K + kb));
    else
      af = bf16x8{};
#pragma unroll
    for (int q = 0; q < 8; ++q) bf[q] = col < rank ? (__bf16)a[(size_t)(kb + q) * rank + col] : (__bf16)0.0f;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf, acc, 0, 0, 0);
  }
  // acc[e] = C[row 4 (lane / 16) + e][col lane % 16]
#pragma unroll
  for (int e = 0; e < 4; ++e) part[w][4 * (lane >> 4) + e][lane & 15] = acc[e];
  __syncthreads();
  const int r = threadIdx.x >> 4, c = threadIdx.x & 15;
  float s = 0.0f;
#pragma unroll
  for (int q = 0; q < kXaWaves; ++q) s += part[q][r][c];
  if (m0 + r < M) xa[(size_t)(m0 + r) * pad + c0 + c] = c0 + c < rank ? s * scaling : 0.0f;
}

}  // namespace

bool gemm_supported(int M, int K, int N, const void* x) {
  // every X offset a workgroup forms, rows past M included, stays below 2^31
  return M > 0 && K >= kBK && K % kBK == 0 && N % kBN == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
         ((uint64_t)M + kBM) * (uint64_t)K * 2u < (1ull << 31);
}

int lora_pad(int rank) { return (rank + 15) / 16 * 16; }

hipError_t launch_lora_xa_bf16(const uint16_t* x, const float* a, int M, int K, int rank, float scaling, float* xa,
                               hipStream_t stream) {
  if (rank < 1 || rank > 64 || K % 32 != 0) return hipErrorInvalidValue;
  const dim3 grid((M + 15) / 16, lora_pad(rank) / 16);
  lora_xa_mfma_kernel<<<grid, 64 * kXaWaves, 0, stream>>>(x, a, M, K, rank, lora_pad(rank), scaling, xa);
  return hipGetLastError();
}

hipError_t launch_gemm(const uint16_t* x, const uint8_t* packed, const ScalesArg& scales, int M, int K, int N,
                       const float* bias, const float* lora_xa, const float* lora_b, int lora_rank, void* y,
                       bool y_bf16, hipStream_t stream) {
  GemmArgs g{};
  g.x = x;
  g.packed = packed;
  g.scales = scales;
  g.M = M;
  g.K = K;
  g.N = N;
  g.bias = bias;
  g.lora_xa = lora_xa;
  g.lora_b = lora_b;
  g.lora_rank = lora_rank;
  g.lora_pad = lora_pad(lora_rank);
  g.y = y;
  g.y_bf16 = y_bf16;
  g.tiles_n = N / kBN;
  const bool dq = scales.kind == kScalesDQ;
  const bool lora = lora_xa != nullptr;
#define UNIFUR_GEMM_CASE(D, B, R) \
  if (dq == D && y_bf16 == B && lora == R) return launch_g<D, B, R>(g, stream);
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

}  // namespace unifur
