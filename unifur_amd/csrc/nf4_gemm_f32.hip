// nf4_gemm_f32.hip -- f32 MFMA GEMM over an NF4 weight dequantized exactly
// into LDS: the linear and its backward for f32 activations (and f32 dY) at
// batch sizes past the skinny kernel's.
//
// Forward: Y[M, N] = X[M, K] deq(W)[K, N] (+ bias) (+ scaling (X A) B), the
// reference's arithmetic for Nf4Linear::forward / QloraLinear::forward
// (src/qwennet.rs:238-241, :325-345): the weight operand is
// NF4_LEVELS[c] * scale in f32 (src/quantize.rs:362, the reference's
// dequantized value bit for bit), products and sums in f32 on
// v_mfma_f32_32x32x2f32.  Backward (TRANS): dX[M, d_in] = dY[M, d_out]
// deq(W)^T (+ scaling (dY B^T) A^T), the autodiff of the same function with
// the base weight frozen (src/qwentrain.rs:421-470).  No weight-sized
// scratch: each workgroup dequantizes the W tiles it needs.
//
// Tiling.  A 256-thread workgroup owns a 128 x 128 output tile, K in steps
// of 32; wave w computes rows 64 (w % 2) and columns 64 (w / 2) as 2 x 2
// MFMA 32x32x2 tiles (64 f32 accumulators).  Each step's X tile [128][32]
// and W tile [32][128] (as B[k][n]) are staged through LDS in two buffers,
// X rows padded to 33 floats and W rows to 160 floats so that an operand
// read (32 consecutive rows of one k, or 32 consecutive columns of k and
// k + 1) touches 64 distinct banks.  The next step's X values and W codes
// are loaded into registers while the current step's MFMAs run, then
// dequantized and written to the other buffer; one barrier per step.
// 78 KiB of LDS: two workgroups per CU.
#include "nf4_gemm_f32.hpp"

#include <atomic>

namespace unifur {
namespace {

constexpr int kFM = 128, kFN = 128, kFK = 32;
constexpr int kFThreads = 256;
constexpr int kXPitch = kFK + 1;         // floats per X row in LDS
constexpr int kWPitch = kFN + 32;        // floats per W row (one k) in LDS
constexpr int kXFloats = kFM * kXPitch;  // 4224
constexpr int kWFloats = kFK * kWPitch;  // 5120
constexpr int kStageFloats = kXFloats + kWFloats;
constexpr int kLutOff = 2 * kStageFloats * 4;  // byte LUT: 256 x {level lo, level hi}
constexpr int kDqOff = kLutOff + 256 * 8;      // DQ scales: 256 x f32
constexpr size_t kF32Smem = kDqOff + 256 * 4;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) const f32x2 lds_f32x2_c;

// One step's global data of this thread, held in registers until the
// MFMAs of the current step have been issued.
struct F32Step {
  f32x4 x[4];       // X rows t / 8 + 32 p, columns 4 (t % 8) .. + 3 of the step
  u32x2 code[2];    // W codes: 16 values (normal: 1 group; TRANS: 1 group, code[1] unused)
  uint32_t scale;   // f32 bits, or the u8 DQ code
  bool wlive;       // the W group lies inside the weight
};

template <bool DQ, bool STRIPED, bool TRANS>
__device__ __forceinline__ void f32_load(F32Step& S, const F32GemmArgs& g, int m0, int n0, int k0, int tid) {
  // X: [M][Kr] f32, Kr % 4 == 0 (a float4 is inside or outside a row)
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int r = tid / 8 + 32 * p, c4 = 4 * (tid % 8);
    const int m = m0 + r, k = k0 + c4;
    S.x[p] = (m < g.M && k < g.K) ? *reinterpret_cast<const f32x4*>(g.x + (size_t)m * g.K + k) : f32x4{};
  }
  // W: 16 consecutive values of one row of the stored weight [wk][wn]
  // (normal: weight row k = k0 + t / 8, columns n0 + 16 (t % 8) ..; TRANS:
  // weight row n = n0 + t / 2, columns k0 + 16 (t % 2) ..)
  const int wrow = TRANS ? n0 + tid / 2 : k0 + tid / 8;
  const int wcol = TRANS ? k0 + 16 * (tid % 2) : n0 + 16 * (tid % 8);
  const int wrows = TRANS ? g.N : g.K, wcols = TRANS ? g.K : g.N;  // the stored weight's d_in, d_out
  S.wlive = wrow < wrows && wcol < wcols;
  if (!S.wlive) return;
  size_t code_byte, scale_idx;
  if constexpr (STRIPED) {
    code_byte = ((size_t)(wcol / 16) * wrows + wrow) * 8;
    scale_idx = (size_t)(wcol / kBlock) * wrows + wrow;
  } else {
    code_byte = (size_t)wrow * (wcols / 2) + wcol / 2;
    scale_idx = (size_t)wrow * (wcols / kBlock) + wcol / kBlock;
  }
  S.code[0] = *reinterpret_cast<const u32x2*>(g.packed + code_byte);
  S.scale = DQ ? (uint32_t)g.scales.dq_codes[scale_idx] : __float_as_uint(g.scales.absmax[scale_idx]);
}

template <bool DQ, bool TRANS>
__device__ __forceinline__ void f32_store(const F32Step& S, unsigned char* smem, int buf, int tid) {
  float* xs = reinterpret_cast<float*>(smem) + buf * kStageFloats;
  float* ws = xs + kXFloats;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int r = tid / 8 + 32 * p, c4 = 4 * (tid % 8);
    lds_f32* d = reinterpret_cast<lds_f32*>((size_t)(xs + r * kXPitch + c4));
    d[0] = S.x[p].x;
    d[1] = S.x[p].y;
    d[2] = S.x[p].z;
    d[3] = S.x[p].w;
  }
  // the 16 weight values level * scale (one f32 multiply, the reference's
  // dequantized value), or zeros past the weight
  const float s = DQ ? reinterpret_cast<const float*>(smem + kDqOff)[S.scale & 0xffu] : __uint_as_float(S.scale);
  float v[16];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t byte = (S.code[0][j >> 2] >> (8 * (j & 3))) & 0xffu;
    const f32x2 l = *reinterpret_cast<lds_f32x2_c*>((size_t)(smem + kLutOff + byte * 8));
    v[2 * j] = S.wlive ? l.x * s : 0.0f;
    v[2 * j + 1] = S.wlive ? l.y * s : 0.0f;
  }
  if constexpr (TRANS) {
    // weight row n (an output column), columns k .. k + 15: B[k + i][n]
    const int n = tid / 2, kk = 16 * (tid % 2);
#pragma unroll
    for (int i = 0; i < 16; ++i) *reinterpret_cast<lds_f32*>((size_t)(ws + (kk + i) * kWPitch + n)) = v[i];
  } else {
    // weight row k, columns 16 (t % 8) .. + 15: B[k][n .. n + 15], 16-byte aligned
    const int k = tid / 8, n = 16 * (tid % 8);
    lds_f32x4* d = reinterpret_cast<lds_f32x4*>((size_t)(ws + k * kWPitch + n));
    d[0] = f32x4{v[0], v[1], v[2], v[3]};
    d[1] = f32x4{v[4], v[5], v[6], v[7]};
    d[2] = f32x4{v[8], v[9], v[10], v[11]};
    d[3] = f32x4{v[12], v[13], v[14], v[15]};
  }
}

template <bool DQ, bool STRIPED, bool TRANS, bool YBF16>
__global__ __launch_bounds__(kFThreads) void gemm_f32_mfma_kernel(F32GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-aware order: workgroup b runs on XCD b % 8; each XCD takes a
  // contiguous run of tiles in row-major (m, n) order (shared X rows)
  const int nb = gridDim.x, b = blockIdx.x;
  const int t = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
  const int tiles_n = (g.N + kFN - 1) / kFN;
  const int m0 = (t / tiles_n) * kFM, n0 = (t % tiles_n) * kFN;

  {
    float* lut = reinterpret_cast<float*>(smem + kLutOff);
    lut[2 * tid] = level(tid & 15);
    lut[2 * tid + 1] = level(tid >> 4);
    if constexpr (DQ) reinterpret_cast<float*>(smem + kDqOff)[tid] = ((float)tid / 255.0f) * (*g.scales.scale_of_scales);
  }
  const int nk = (g.K + kFK - 1) / kFK;
  F32Step S;
  f32_load<DQ, STRIPED, TRANS>(S, g, m0, n0, 0, tid);
  __syncthreads();  // LUTs
  f32_store<DQ, TRANS>(S, smem, 0, tid);
  __syncthreads();

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  const int arow = 64 * wm + (lane & 31), bcol = 64 * wn + (lane & 31), kl = lane >> 5;
  for (int s = 0; s < nk; ++s) {
    const int buf = s & 1;
    if (s + 1 < nk) f32_load<DQ, STRIPED, TRANS>(S, g, m0, n0, (s + 1) * kFK, tid);
    const float* xs = reinterpret_cast<const float*>(smem) + buf * kStageFloats;
    const float* ws = xs + kXFloats;
#pragma unroll
    for (int k2 = 0; k2 < kFK / 2; ++k2) {
      const int k = 2 * k2 + kl;
      float a[2], bb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const lds_f32*>((size_t)(xs + (arow + 32 * i) * kXPitch + k));
#pragma unroll
      for (int j = 0; j < 2; ++j) bb[j] = *reinterpret_cast<const lds_f32*>((size_t)(ws + k * kWPitch + bcol + 32 * j));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], bb[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < nk) f32_store<DQ, TRANS>(S, smem, buf ^ 1, tid);
    __syncthreads();
  }

  // the adapter: acc += (xa scaling) B over the rank, on the same MFMAs; xa
  // [M][lora_ld] f32 and B element (j, n) at lora_b[j sbj + n sbn]
  if (g.lora_xa) {
    for (int j0 = 0; j0 < g.lora_rank; j0 += 2) {
      const int j = j0 + kl;
      const bool jl = j < g.lora_rank;
      float a[2], bb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int m = m0 + arow + 32 * i;
        a[i] = (jl && m < g.M) ? g.lora_xa[(size_t)m * g.lora_ld + j] * g.lora_scaling : 0.0f;
      }
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int n = n0 + bcol + 32 * jj;
        bb[jj] = (jl && n < g.N) ? g.lora_b[(size_t)j * g.lora_sbj + (size_t)n * g.lora_sbn] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], bb[jj], acc[i][jj], 0, 0, 0);
    }
  }
  // acc[i][j][4 a + e] is C[row 32 i + 8 a + 4 (lane / 32) + e][col 32 j +
  // lane % 32] of the wave's tile: each store instruction writes 32
  // consecutive columns of two rows
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + bcol + 32 * j;
    if (n >= g.N) continue;
    const float bias = g.bias ? g.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * kl + (r & 3);
        if (m >= g.M) continue;
        const float y = acc[i][j][r] + bias;
        if constexpr (YBF16)
          reinterpret_cast<uint16_t*>(g.y)[(size_t)m * g.N + n] = (uint16_t)(pack_bf16x2(y, 0.0f) & 0xffffu);
        else
          reinterpret_cast<float*>(g.y)[(size_t)m * g.N + n] = y;
      }
  }
}

template <bool DQ, bool STRIPED, bool TRANS, bool YBF16>
hipError_t launch_f(const F32GemmArgs& g, hipStream_t stream) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  const void* fn = reinterpret_cast<const void*>(&gemm_f32_mfma_kernel<DQ, STRIPED, TRANS, YBF16>);
  if (!(done.load(std::memory_order_acquire) & bit)) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kF32Smem);
    if (e != hipSuccess) return e;
    done.fetch_or(bit, std::memory_order_acq_rel);
  }
  const int tiles = ((g.M + kFM - 1) / kFM) * ((g.N + kFN - 1) / kFN);
  gemm_f32_mfma_kernel<DQ, STRIPED, TRANS, YBF16><<<tiles, kFThreads, kF32Smem, stream>>>(g);
  return hipGetLastError();
}

}  // namespace

bool gemm_f32_mfma_supported(int M, int Kr, int N, int w_d_out, const void* x) {
  // the reduction dim a multiple of 4 (whole float4 loads), the stored
  // weight's d_out of 64 (whole blocks along a row), 16-byte aligned X
  return M > 0 && Kr > 0 && N > 0 && Kr % 4 == 0 && w_d_out % 64 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (((uint64_t)M + kFM) * (uint64_t)(Kr) < (1ull << 40));
}

hipError_t launch_gemm_f32_mfma(const F32GemmArgs& g, bool dq, bool striped, bool trans, bool y_bf16,
                                hipStream_t stream) {
#define UNIFUR_F32_CASE(D, S, T, B) \
  if (dq == D && striped == S && trans == T && y_bf16 == B) return launch_f<D, S, T, B>(g, stream);
  UNIFUR_F32_CASE(true, true, false, false)
  UNIFUR_F32_CASE(true, true, false, true)
  UNIFUR_F32_CASE(true, false, false, false)
  UNIFUR_F32_CASE(true, false, false, true)
  UNIFUR_F32_CASE(false, true, false, false)
  UNIFUR_F32_CASE(false, true, false, true)
  UNIFUR_F32_CASE(false, false, false, false)
  UNIFUR_F32_CASE(false, false, false, true)
  UNIFUR_F32_CASE(true, true, true, false)
  UNIFUR_F32_CASE(true, true, true, true)
  UNIFUR_F32_CASE(true, false, true, false)
  UNIFUR_F32_CASE(true, false, true, true)
  UNIFUR_F32_CASE(false, true, true, false)
  UNIFUR_F32_CASE(false, true, true, true)
  UNIFUR_F32_CASE(false, false, true, false)
  UNIFUR_F32_CASE(false, false, true, true)
#undef UNIFUR_F32_CASE
  return hipErrorInvalidValue;
}

}  // namespace unifur
