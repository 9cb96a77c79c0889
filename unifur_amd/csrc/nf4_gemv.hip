// nf4_gemv.hip -- bandwidth-bound NF4-weight linear for decode (few rows).
//
// Computes y[t][o] = sum_i x[t][i] * deq(W)[i][o] (+ bias[o]) with W the
// reference's packed [d_in, d_out] row-major weight (src/qwennet.rs:161-241:
// Nf4Linear::forward = dequantize, then burn linear).  The weight is never
// materialised: each 16-byte load of packed codes (32 output columns of one
// input row) is expanded in registers.
//
// Work split.  A workgroup owns a 256-column tile and a slab of input rows.
// Lane (tid % 8) of a row group reads bytes [16 l, 16 l + 16) of the tile's
// 128-byte row segment, so a wave reads eight whole 128-byte lines per load,
// and every thread issues all of its loads before it touches any of them.
// Partial column sums are reduced across the workgroup's 32 row groups in
// LDS, then across row slabs (split-K) in a fixed order by the last
// workgroup to finish a tile (a per-tile arrival counter in the workspace),
// which also applies bias, the optional LoRA term and the output
// conversion.  Results are deterministic run to run.
//
// Decode arithmetic.  Per (row, 64-block) the activation is folded with the
// block scale once, xs = x[i] * scale; every code byte then costs one
// v_perm_b32 (builds the LDS address of its LUT entry), one ds_read_b64
// ({level[lo], level[hi]}) and two FMAs.  The 256-entry byte LUT is
// replicated 32 times with an entry stride of 256 bytes, so lane l always
// reads copy (l % 32): any 32 consecutive lanes hit 32 distinct bank pairs.
//
// PAIR mode computes gate and up of a SwiGLU block in one pass over the same
// x and writes silu(gate) * up (src/qwennet.rs:816-819, src/tensor_ext.rs:87-90).
#include "nf4_gemv.hpp"

#include <atomic>

namespace unifur {
namespace {

constexpr int kLanesPerRow = 8;
constexpr int kTileCols = kLanesPerRow * 32;  // 256 output columns per workgroup
constexpr int kGemvThreads = 256;
constexpr int kRowGroups = kGemvThreads / kLanesPerRow;  // 32 rows per step
constexpr int kLutCopies = 32;
constexpr int kLutBytes = 256 * kLutCopies * 8;  // 64 KiB
constexpr int kChunkStride = 32 + 4;             // floats; padded per 32-column chunk
constexpr int kRedRowStride = kLanesPerRow * kChunkStride;
constexpr int kRedBytes = kRowGroups * kRedRowStride * 4;
static_assert(kRedBytes <= kLutBytes, "reduction buffer reuses the LUT space");
// byte LUT | DQ LUT of weight 0 | DQ LUT of weight 1 | last-arrival flag
constexpr size_t kGemvSmem = kLutBytes + 2 * 256 * sizeof(float) + 16;

struct GemvArgs {
  const void* x;  // [rows, d_in] f32 or bf16
  int rows;
  int d_in;
  int rows_per_wg;  // input rows per workgroup (kRowGroups * RT)
  int splits;       // gridDim.y
  int nweights;
  GemvWeight w[kMaxGemvWeights];
  int tile_begin[kMaxGemvWeights + 1];  // prefix sums of column tiles per weight
};

__device__ __forceinline__ float silu_f32(float z) { return z * (1.0f / (1.0f + __expf(-z))); }

// One weight's loads for this thread: RT rows of 16 code bytes and a scale.
template <int RT, bool DQ>
struct RowLoads {
  u32x4 code[RT];
  uint32_t scale[RT];  // f32 absmax bits, or (DQ) the u8 scale code
};

template <int RT, bool DQ>
__device__ __forceinline__ void issue_loads(RowLoads<RT, DQ>& L, const GemvWeight& W, int k0, int K, int n0,
                                            bool col_ok) {
  const int N = W.d_out;
  const size_t row_bytes = (size_t)N / 2;
  const size_t blocks_per_row = (size_t)N / kBlock;
  const uint8_t* cp = W.packed + (size_t)k0 * row_bytes + n0 / 2;
  const size_t b0 = (size_t)k0 * blocks_per_row + n0 / kBlock;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const bool ok = col_ok && (k0 + r * kRowGroups) < K;
    const size_t roff = (size_t)r * kRowGroups;
    L.code[r] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cp + roff * row_bytes))
                   : u32x4{0u, 0u, 0u, 0u};
    if constexpr (DQ)
      L.scale[r] = ok ? (uint32_t)W.scales.dq_codes[b0 + roff * blocks_per_row] : 0u;
    else
      L.scale[r] = ok ? __float_as_uint(W.scales.absmax[b0 + roff * blocks_per_row]) : 0u;
  }
}

template <int T, int RT, bool DQ>
__device__ __forceinline__ void accumulate(float (&acc)[T][32], const RowLoads<RT, DQ>& L, const float (&xv)[T][RT],
                                           const unsigned char* smem, const float* dq_lut, uint32_t lane_off) {
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    // rows out of range carry x = 0 and code 0 (level -1): they add 0.
    const float s = DQ ? dq_lut[L.scale[r]] : __uint_as_float(L.scale[r]);
    float xs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) xs[t] = xv[t][r] * s;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t w = L.code[r][d];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // LDS byte address = (byte j of w) << 8 | lane_off
        const uint32_t addr = perm_b32(w, lane_off, 0x0c0c0000u | ((4u + j) << 8));
        const f32x2 lv = *reinterpret_cast<const f32x2*>(smem + addr);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          acc[t][8 * d + 2 * j] = __builtin_fmaf(xs[t], lv.x, acc[t][8 * d + 2 * j]);
          acc[t][8 * d + 2 * j + 1] = __builtin_fmaf(xs[t], lv.y, acc[t][8 * d + 2 * j + 1]);
        }
      }
    }
    // Keep the scheduler from hoisting every row's LDS reads (register blow-up).
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Sum the 32 row groups' partial columns; thread tid gets column tid.
template <int T>
__device__ __forceinline__ void reduce_rows(float (&out)[T], const float (&acc)[T][32], float* red, int rg, int lir,
                                           int tid) {
  const int ccol = (tid / 32) * kChunkStride + (tid % 32);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    __syncthreads();
    f32x4* dst = reinterpret_cast<f32x4*>(red + rg * kRedRowStride + lir * kChunkStride);
#pragma unroll
    for (int q = 0; q < 8; ++q) dst[q] = f32x4{acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
    __syncthreads();
    float sum = 0.0f;
#pragma unroll 8
    for (int g = 0; g < kRowGroups; ++g) sum += red[g * kRedRowStride + ccol];
    out[t] = sum;
  }
}

__device__ __forceinline__ float epilogue_value(const GemvWeight& W, float base, int t, int gcol) {
  float y = base;
  if (W.bias) y += W.bias[gcol];
  if (W.lora_xa) {
    // base(x) + ((x A) B) * scaling (src/qwennet.rs:325-344, src/quantize.rs:619-624)
    float l = 0.0f;
    for (int j = 0; j < W.lora_rank; ++j)
      l = __builtin_fmaf(W.lora_xa[t * W.lora_rank + j], W.lora_b[(size_t)j * W.d_out + gcol], l);
    y += l * W.lora_scaling;
  }
  return y;
}

__device__ __forceinline__ void store_y(const GemvWeight& W, size_t idx, float y) {
  if (W.y_bf16)
    reinterpret_cast<uint16_t*>(W.y)[idx] = (uint16_t)(pack_bf16x2(y, 0.0f) & 0xffffu);
  else
    reinterpret_cast<float*>(W.y)[idx] = y;
}

template <int T, int RT, bool XBF16, bool DQ, bool PAIR>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* dq_lut = reinterpret_cast<float*>(smem + kLutBytes);
  int& s_is_last = *reinterpret_cast<int*>(smem + kLutBytes + 2 * 256 * sizeof(float));

  int wi = 0;
  if constexpr (!PAIR) {
#pragma unroll
    for (int i = 1; i < kMaxGemvWeights; ++i)
      if (i < a.nweights && (int)blockIdx.x >= a.tile_begin[i]) wi = i;
  }
  const GemvWeight& W = a.w[wi];
  const int tile = blockIdx.x - a.tile_begin[wi];
  const int N = W.d_out;
  const int K = a.d_in;
  const int tid = threadIdx.x;
  const int lir = tid % kLanesPerRow;
  const int rg = tid / kLanesPerRow;
  const int n0 = tile * kTileCols + lir * 32;
  const bool col_ok = n0 < N;
  const int k0 = blockIdx.y * a.rows_per_wg + rg;

  // ---- every global load first ------------------------------------------------
  RowLoads<RT, DQ> L0;
  issue_loads<RT, DQ>(L0, W, k0, K, n0, col_ok);
  RowLoads<PAIR ? RT : 1, DQ> L1;
  if constexpr (PAIR) issue_loads<RT, DQ>(L1, a.w[1], k0, K, n0, col_ok);
  float xv[T][RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int k = k0 + r * kRowGroups;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const size_t idx = (size_t)t * K + k;
      float v = 0.0f;
      if (k < K) {
        if constexpr (XBF16)
          v = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.x)[idx]);
        else
          v = reinterpret_cast<const float*>(a.x)[idx];
      }
      xv[t][r] = v;
    }
  }

  // ---- LUTs (built while the loads are in flight) ----------------------------------
  {
    const float lo = level(tid & 15), hi = level(tid >> 4);
    const f32x4 v = {lo, hi, lo, hi};
    f32x4* dst = reinterpret_cast<f32x4*>(smem + tid * (kLutCopies * 8));
#pragma unroll
    for (int c = 0; c < kLutCopies / 2; ++c) dst[c] = v;
    if constexpr (DQ) {
      // ((float)q / 255.0f) * scale_of_scales (src/quantize.rs:349), per code q
      dq_lut[tid] = ((float)tid / 255.0f) * (*W.scales.scale_of_scales);
      if constexpr (PAIR) dq_lut[256 + tid] = ((float)tid / 255.0f) * (*a.w[1].scales.scale_of_scales);
    }
  }
  __syncthreads();

  // ---- decode + accumulate ------------------------------------------------------
  const uint32_t lane_off = (uint32_t)(tid & 31) * 8u;
  float* red = reinterpret_cast<float*>(smem);
  float res0[T];
  float res1[T];
  {
    float acc0[T][32];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < 32; ++i) acc0[t][i] = 0.0f;
    accumulate<T, RT, DQ>(acc0, L0, xv, smem, dq_lut, lane_off);
    if constexpr (PAIR) {
      float acc1[T][32];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 32; ++i) acc1[t][i] = 0.0f;
      accumulate<T, RT, DQ>(acc1, L1, xv, smem, dq_lut + 256, lane_off);
      reduce_rows<T>(res0, acc0, red, rg, lir, tid);
      reduce_rows<T>(res1, acc1, red, rg, lir, tid);
    } else {
      reduce_rows<T>(res0, acc0, red, rg, lir, tid);
    }
  }

  const int gcol = tile * kTileCols + tid;
  const bool gcol_ok = gcol < N;
  if (a.splits > 1) {
    if (gcol_ok) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        W.partials[((size_t)blockIdx.y * a.rows + t) * N + gcol] = res0[t];
        if constexpr (PAIR) a.w[1].partials[((size_t)blockIdx.y * a.rows + t) * N + gcol] = res1[t];
      }
    }
    // Release the partials, count arrivals; the last arrival reduces in order.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(&W.counters[tile], 1u);
      s_is_last = (prev == (unsigned)(a.splits - 1));
    }
    __syncthreads();
    if (!s_is_last) return;
    __threadfence();
    if (gcol_ok) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        float s0 = 0.0f, s1 = 0.0f;
        for (int s = 0; s < a.splits; ++s) {
          const size_t idx = ((size_t)s * a.rows + t) * N + gcol;
          s0 += __builtin_nontemporal_load(&W.partials[idx]);
          if constexpr (PAIR) s1 += __builtin_nontemporal_load(&a.w[1].partials[idx]);
        }
        res0[t] = s0;
        if constexpr (PAIR) res1[t] = s1;
      }
    }
    if (tid == 0) W.counters[tile] = 0u;  // leave the workspace zeroed for the next call
  }

  if (!gcol_ok) return;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float y = epilogue_value(W, res0[t], t, gcol);
    if constexpr (PAIR) {
      const float u = epilogue_value(a.w[1], res1[t], t, gcol);
      y = silu_f32(y) * u;  // silu(gate(x)) * up(x)
    }
    store_y(W, (size_t)t * N + gcol, y);
  }
}

template <int T, int RT, bool XBF16, bool DQ, bool PAIR>
hipError_t launch_t(const GemvArgs& a, int grid_x, hipStream_t stream) {
  // Dynamic LDS above 64 KiB needs the attribute, once per device.
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  const void* fn = reinterpret_cast<const void*>(&gemv_kernel<T, RT, XBF16, DQ, PAIR>);
  if (!(done.load(std::memory_order_acquire) & bit)) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvSmem);
    if (e != hipSuccess) return e;
    done.fetch_or(bit, std::memory_order_acq_rel);
  }
  gemv_kernel<T, RT, XBF16, DQ, PAIR><<<dim3(grid_x, a.splits), kGemvThreads, kGemvSmem, stream>>>(a);
  return hipGetLastError();
}

template <int T, int RT, bool PAIR>
hipError_t dispatch_flags(const GemvArgs& a, int grid_x, bool xbf16, bool dq, hipStream_t stream) {
  if (xbf16) return dq ? launch_t<T, RT, true, true, PAIR>(a, grid_x, stream)
                       : launch_t<T, RT, true, false, PAIR>(a, grid_x, stream);
  return dq ? launch_t<T, RT, false, true, PAIR>(a, grid_x, stream)
            : launch_t<T, RT, false, false, PAIR>(a, grid_x, stream);
}

int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace

GemvPlan plan_gemv(int rows, int d_in, const int* d_out, int nweights, bool pair) {
  GemvPlan p{};
  int tiles = 0;
  const int nw_tiles = pair ? 1 : nweights;
  for (int i = 0; i < nw_tiles; ++i) tiles += ceil_div(d_out[i], kTileCols);
  // Rows per thread: 16 for one activation row, 8 otherwise, halved in PAIR
  // mode (register budget); then halved while the grid has fewer than 512
  // workgroups (two resident per CU on 256 CUs, every load issued up front).
  // Rows per thread: 16 for one activation row, else 8 (register budget), 4
  // in PAIR mode; halved while the grid has fewer than 512 workgroups (two
  // resident per CU on 256 CUs, every load issued up front).
  int rt = pair ? 4 : (rows <= 1 ? 16 : 8);
  while (rt > 4 && (long)tiles * ceil_div(d_in, kRowGroups * rt) < 512) rt /= 2;
  p.rows_per_thread = rt;
  p.rows_per_wg = kRowGroups * rt;
  p.splits = ceil_div(d_in, p.rows_per_wg);
  p.tiles = tiles;
  p.pair = pair;
  for (int i = 0; i < nweights; ++i) {
    p.counter_count[i] = ceil_div(d_out[i], kTileCols);
    p.partial_count[i] = p.splits > 1 ? (size_t)p.splits * rows * d_out[i] : 0;
  }
  return p;
}

hipError_t launch_gemv(const GemvPlan& p, const void* x, bool x_bf16, int rows, int d_in, const GemvWeight* weights,
                       int nweights, hipStream_t stream) {
  GemvArgs a{};
  a.x = x;
  a.rows = rows;
  a.d_in = d_in;
  a.rows_per_wg = p.rows_per_wg;
  a.splits = p.splits;
  a.nweights = nweights;
  int t = 0;
  for (int i = 0; i < nweights; ++i) {
    a.w[i] = weights[i];
    a.tile_begin[i] = p.pair ? 0 : t;
    if (!p.pair || i == 0) t += ceil_div(weights[i].d_out, kTileCols);
  }
  for (int i = nweights; i <= kMaxGemvWeights; ++i) a.tile_begin[i] = t;
  const bool dq = weights[0].scales.kind == kScalesDQ;
  const int grid_x = t;
  const int rt = p.rows_per_thread;
  if (p.pair) {
    if (rows == 1) return dispatch_flags<1, 4, true>(a, grid_x, x_bf16, dq, stream);
    if (rows == 2) return dispatch_flags<2, 4, true>(a, grid_x, x_bf16, dq, stream);
    return hipErrorInvalidValue;
  }
#define UNIFUR_GEMV_ROWS(TT)                                                          \
  case TT:                                                                            \
    if (rt == 8) return dispatch_flags<TT, 8, false>(a, grid_x, x_bf16, dq, stream); \
    return dispatch_flags<TT, 4, false>(a, grid_x, x_bf16, dq, stream);
  switch (rows) {
    case 1:
      if (rt == 16) return dispatch_flags<1, 16, false>(a, grid_x, x_bf16, dq, stream);
      if (rt == 8) return dispatch_flags<1, 8, false>(a, grid_x, x_bf16, dq, stream);
      return dispatch_flags<1, 4, false>(a, grid_x, x_bf16, dq, stream);
    UNIFUR_GEMV_ROWS(2)
    UNIFUR_GEMV_ROWS(3)
    UNIFUR_GEMV_ROWS(4)
    default:
      return hipErrorInvalidValue;
  }
#undef UNIFUR_GEMV_ROWS
}

}  // namespace unifur
