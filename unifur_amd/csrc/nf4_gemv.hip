// nf4_gemv.hip -- bandwidth-bound NF4-weight linear for decode (few rows).
//
// Computes y[t][o] = sum_i x[t][i] * deq(W)[i][o] (+ bias[o]) with W the
// reference's packed [d_in, d_out] row-major weight (src/qwennet.rs:161-241:
// Nf4Linear::forward = dequantize, then burn linear).  The weight is never
// materialised: each 16-byte load of packed codes (32 output columns of one
// input row) is expanded in registers.
//
// Decode arithmetic (both kernels).  Per (row, 64-block) the activation is
// folded with the block scale once, xs = x[i] * scale; every code byte then
// costs one v_perm_b32 (builds the LDS address of its LUT entry), one
// ds_read_b64 ({level[lo], level[hi]}) and two FMAs.  The 256-entry byte LUT
// is replicated 32 times with an entry stride of 256 bytes, so lane l always
// reads copy (l % 32): any 32 consecutive lanes hit 32 distinct bank pairs.
// Every thread issues all of its global loads before the LUT is built, and
// consumes them row by row as they arrive.
//
// Work split.  A 512-thread workgroup owns a 256-column tile and a slab of
// input rows.  Lane (tid % 8) of a row group reads bytes [16 l, 16 l + 16)
// of the tile's 128-byte row segment, so a wave reads eight whole 128-byte
// lines per load instruction.  (Narrower per-workgroup strips would let one
// workgroup own all rows of its columns, but then every lane of a load
// touches a different line and the L2-to-CU traffic grows eightfold.)
// Partial column sums are reduced across the workgroup's row groups in LDS,
// then across row slabs (split-K) by the last workgroup to finish the tile
// (a per-tile arrival counter in the workspace), which reduces them in a
// fixed order: results are deterministic run to run.
//
// PAIR mode computes gate and up of a SwiGLU block in one pass over the same
// x and writes silu(gate) * up (src/qwennet.rs:816-819, src/tensor_ext.rs:87-90).
#include "nf4_gemv.hpp"

#include <atomic>

namespace unifur {
namespace {

constexpr int kThreads = 512;
constexpr int kLanesPerRow = 8;
constexpr int kTileCols = kLanesPerRow * 32;         // 256 output columns per workgroup
constexpr int kRowGroups = kThreads / kLanesPerRow;  // 64 input rows per step
constexpr int kChunkStride = 32 + 4;                 // floats; padded per 32-column chunk
constexpr int kRedRowStride = kLanesPerRow * kChunkStride;
constexpr int kLutCopies = 32;
constexpr int kLutBytes = 256 * kLutCopies * 8;  // 64 KiB
// LDS: byte LUT | DQ LUT of weight 0 | DQ LUT of weight 1 | 16 levels, all
// dead once the rows are accumulated, when the row-group reduction buffer
// (64 groups x 288 floats) reuses the space; the last-arrival flag follows.
constexpr int kDqLutOffset = kLutBytes;
constexpr int kLevelsOffset = kDqLutOffset + 2 * 256 * 4;
constexpr int kRedBytes = kRowGroups * kRedRowStride * 4;
static_assert(kRedBytes >= kLevelsOffset + 16 * 4, "reduction buffer covers the LUT space");
constexpr int kFlagOffset = kRedBytes;
constexpr size_t kGemvSmem = kFlagOffset + 16;  // 72 KiB: two workgroups per CU

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

typedef __attribute__((address_space(3))) const f32x2 lds_f32x2;

__device__ __forceinline__ float silu_f32(float z) { return z * (1.0f / (1.0f + __expf(-z))); }

// One weight's loads for this thread: RT rows of 16 code bytes and a scale.
template <int RT>
struct RowLoads {
  u32x4 code[RT];
  uint32_t scale[RT];  // f32 absmax bits, or (DQ) the u8 scale code
};

// Buffer resources bound each workgroup's loads to its own row slab: a load
// past the slab (or past the tensor) returns zero from the hardware bounds
// check instead of touching memory, so no address needs clamping and no
// other slab's bytes are fetched.  Word 3 is the raw-buffer descriptor.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

// Rows k0 + r * RS of the slab ending at row ke.  Loads are issued
// unconditionally and are not touched until after the LUT barrier: a load
// under a branch, or any use of a loaded value before that barrier, would
// make the wave wait for its whole vector-memory queue there.  Rows past the
// slab read as zero and are cancelled through their activation (xs = 0) in
// accumulate(); lanes past d_out only feed columns that are never stored.
template <int RT, int RS, bool DQ>
__device__ __forceinline__ void issue_loads(RowLoads<RT>& L, const GemvWeight& W, int k0, int ke, int byte0,
                                            int blk0) {
  const uint32_t row_bytes = (uint32_t)W.d_out / 2;
  const uint32_t blocks_per_row = (uint32_t)W.d_out / kBlock;
  const __amdgpu_buffer_rsrc_t codes = make_rsrc(W.packed, (uint32_t)ke * row_bytes);
  const uint32_t c0 = (uint32_t)k0 * row_bytes + (uint32_t)byte0;
  const uint32_t s0 = (uint32_t)k0 * blocks_per_row + (uint32_t)blk0;
#pragma unroll
  for (int r = 0; r < RT; ++r)
    L.code[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               codes, c0 + (uint32_t)(r * RS) * row_bytes, 0, 0));
  if constexpr (DQ) {
    const __amdgpu_buffer_rsrc_t sc = make_rsrc(W.scales.dq_codes, (uint32_t)ke * blocks_per_row);
#pragma unroll
    for (int r = 0; r < RT; ++r)
      L.scale[r] = __builtin_amdgcn_raw_buffer_load_b8(sc, s0 + (uint32_t)(r * RS) * blocks_per_row, 0, 0);
  } else {
    const __amdgpu_buffer_rsrc_t sc = make_rsrc(W.scales.absmax, (uint32_t)ke * blocks_per_row * 4u);
#pragma unroll
    for (int r = 0; r < RT; ++r)
      L.scale[r] = __builtin_amdgcn_raw_buffer_load_b32(sc, 4u * (s0 + (uint32_t)(r * RS) * blocks_per_row), 0, 0);
  }
}

// x[t][k0 + r * RS]; entries past the tensor read as zero (rows past the
// slab are cancelled in accumulate()).
template <int T, int RT, int RS, bool XBF16>
__device__ __forceinline__ void load_x(float (&xv)[T][RT], const void* x, int k0, int K) {
  const uint32_t esize = XBF16 ? 2u : 4u;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)(T * K) * esize);
#pragma unroll
  for (int r = 0; r < RT; ++r) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t off = ((uint32_t)t * (uint32_t)K + (uint32_t)(k0 + r * RS)) * esize;
      if constexpr (XBF16)
        xv[t][r] = bf16_bits_to_f32(__builtin_amdgcn_raw_buffer_load_b16(xr, off, 0, 0));
      else
        xv[t][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, off, 0, 0));
    }
  }
}

// Byte LUT (and the DQ scale LUTs) in LDS; ends with a barrier.
template <bool DQ, bool PAIR>
__device__ __forceinline__ void build_luts(unsigned char* smem, int tid, const GemvWeight& w0, const GemvWeight& w1) {
  float* dq_lut = reinterpret_cast<float*>(smem + kDqLutOffset);
  // The 16 levels are staged in LDS from immediates (thread 0), so that no
  // LUT value waits on the vector-memory queue holding the weight loads.
  float* lv16 = reinterpret_cast<float*>(smem + kLevelsOffset);
  if (tid == 0) {
#pragma unroll
    for (int c = 0; c < 16; ++c) lv16[c] = __uint_as_float(level_bits(c));
  }
  __syncthreads();
  // entry e = tid % 256 holds {level[e & 15], level[e >> 4]} in 32 copies
  // (16 chunks of 16 bytes); each half of the workgroup writes 8 chunks,
  // rotated by lane so that 8 consecutive lanes hit 8 distinct bank groups.
  const int e = tid & 255, half = tid >> 8;
  const float lo = lv16[e & 15], hi = lv16[e >> 4];
  const f32x4 v = {lo, hi, lo, hi};
  f32x4* dst = reinterpret_cast<f32x4*>(smem + e * (kLutCopies * 8));
#pragma unroll
  for (int j = 0; j < 8; ++j) dst[half * 8 + ((j + tid) & 7)] = v;
  if constexpr (DQ) {
    // ((float)q / 255.0f) * scale_of_scales (src/quantize.rs:349), per code q
    if (half == 0) dq_lut[e] = ((float)e / 255.0f) * (*w0.scales.scale_of_scales);
    if constexpr (PAIR)
      if (half == 1) dq_lut[256 + e] = ((float)e / 255.0f) * (*w1.scales.scale_of_scales);
  }
  // nothing that consumes a weight load may be hoisted above this barrier
  // (it would make every wave wait for its whole load queue here)
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
}

template <int T, int RT, int RS, bool DQ>
__device__ __forceinline__ void accumulate(float (&acc)[T][32], const RowLoads<RT>& L, const float (&xv)[T][RT],
                                           const float* dq_lut, uint32_t lane_off, int k0, int ke) {
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const float s = DQ ? dq_lut[L.scale[r] & 0xffu] : __uint_as_float(L.scale[r]);
    const bool row_ok = k0 + r * RS < ke;
    float xs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) xs[t] = row_ok ? xv[t][r] * s : 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t w = L.code[r][d];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // LDS byte address = (byte j of w) << 8 | lane_off.  The LUT sits at
        // LDS address 0 (the kernels have no static LDS, so dynamic LDS starts
        // there), which lets the address feed ds_read_b64 directly.
        const uint32_t addr = perm_b32(w, lane_off, 0x0c0c0000u | ((4u + j) << 8));
        const f32x2 lv = *reinterpret_cast<const lds_f32x2*>((size_t)addr);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          acc[t][8 * d + 2 * j] = __builtin_fmaf(xs[t], lv.x, acc[t][8 * d + 2 * j]);
          acc[t][8 * d + 2 * j + 1] = __builtin_fmaf(xs[t], lv.y, acc[t][8 * d + 2 * j + 1]);
        }
      }
    }
    // Keep the compiler (IR passes and the machine scheduler) from hoisting
    // every row's LDS reads ahead of this row's FMAs: that needs 2 registers
    // per byte of the whole slab and spills.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
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

// =========================================================== split-K kernel ==

// Sum the 64 row groups' partial columns in LDS: threads 2c and 2c + 1 add
// half of column c's groups each and combine; the even thread holds it.
template <int T>
__device__ __forceinline__ void reduce_rows(float (&out)[T], const float (&acc)[T][32], float* red, int rg, int lir,
                                           int tid) {
  const int col = tid >> 1, half = tid & 1;
  const int ccol = (col / 32) * kChunkStride + (col % 32);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    __syncthreads();
    f32x4* dst = reinterpret_cast<f32x4*>(red + rg * kRedRowStride + lir * kChunkStride);
#pragma unroll
    for (int q = 0; q < 8; ++q) dst[q] = f32x4{acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
    __syncthreads();
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < kRowGroups / 2; ++g) sum += red[(half * (kRowGroups / 2) + g) * kRedRowStride + ccol];
    out[t] = sum + __shfl_xor(sum, 1);
  }
}

// The last arrival's sum over the slabs' partials: all loads of a batch of
// 8 are issued before the first add, and they are added in slab order.
__device__ __forceinline__ float sum_partials(const float* p, size_t stride, int splits) {
  float s = 0.0f;
  for (int s0 = 0; s0 < splits; s0 += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = s0 + i < splits ? load_coherent(p + (size_t)(s0 + i) * stride) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[i];
  }
  return s;
}

template <int T, int RT, bool XBF16, bool DQ, bool PAIR>
__global__ __launch_bounds__(kThreads) void gemv_splitk_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  int& s_is_last = *reinterpret_cast<int*>(smem + kFlagOffset);

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
  const int nn = n0 < N ? n0 : 0;  // lanes past d_out read column 0 and are never stored
  const int kb = blockIdx.y * a.rows_per_wg;
  const int ke = kb + a.rows_per_wg < K ? kb + a.rows_per_wg : K;  // this slab: rows [kb, ke)
  const int k0 = kb + rg;

  float xv[T][RT];
  load_x<T, RT, kRowGroups, XBF16>(xv, a.x, k0, K);
  RowLoads<RT> L0;
  issue_loads<RT, kRowGroups, DQ>(L0, W, k0, ke, nn / 2, nn / kBlock);
  RowLoads<PAIR ? RT : 1> L1;
  if constexpr (PAIR) issue_loads<RT, kRowGroups, DQ>(L1, a.w[1], k0, ke, nn / 2, nn / kBlock);

  build_luts<DQ, PAIR>(smem, tid, W, a.w[PAIR ? 1 : 0]);

  const float* dq_lut = reinterpret_cast<const float*>(smem + kDqLutOffset);
  const uint32_t lane_off = (uint32_t)(tid & 31) * 8u;
  float* red = reinterpret_cast<float*>(smem);
  float res0[T], res1[T];
  {
    float acc0[T][32];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < 32; ++i) acc0[t][i] = 0.0f;
    accumulate<T, RT, kRowGroups, DQ>(acc0, L0, xv, dq_lut, lane_off, k0, ke);
    if constexpr (PAIR) {
      float acc1[T][32];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 32; ++i) acc1[t][i] = 0.0f;
      accumulate<T, RT, kRowGroups, DQ>(acc1, L1, xv, dq_lut + 256, lane_off, k0, ke);
      reduce_rows<T>(res0, acc0, red, rg, lir, tid);
      reduce_rows<T>(res1, acc1, red, rg, lir, tid);
    } else {
      reduce_rows<T>(res0, acc0, red, rg, lir, tid);
    }
  }

  const int gcol = tile * kTileCols + (tid >> 1);
  const bool gcol_ok = (tid & 1) == 0 && gcol < N;
  if (a.splits > 1) {
    if (gcol_ok) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const size_t idx = ((size_t)blockIdx.y * a.rows + t) * N + gcol;
        store_coherent(&W.partials[idx], res0[t]);
        if constexpr (PAIR) store_coherent(&a.w[1].partials[idx], res1[t]);
      }
    }
    wait_all_memory();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&W.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_is_last = (prev == (unsigned)(a.splits - 1));
    }
    __syncthreads();
    if (!s_is_last) return;
    if (gcol_ok) {
      const size_t stride = (size_t)a.rows * N;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        res0[t] = sum_partials(&W.partials[(size_t)t * N + gcol], stride, a.splits);
        if constexpr (PAIR) res1[t] = sum_partials(&a.w[1].partials[(size_t)t * N + gcol], stride, a.splits);
      }
    }
    // leave the counter zeroed for the next call on this workspace
    if (tid == 0) __hip_atomic_store(&W.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (!gcol_ok) return;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float y = epilogue_value(W, res0[t], t, gcol);
    if constexpr (PAIR) y = silu_f32(y) * epilogue_value(a.w[1], res1[t], t, gcol);  // silu(gate x) * up x
    store_y(W, (size_t)t * N + gcol, y);
  }
}

// ================================================================ launching ==

template <typename F>
hipError_t ensure_lds_attribute(F* fn) {
  // Dynamic LDS above 64 KiB needs the attribute, once per device.
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(done.load(std::memory_order_acquire) & bit)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)kGemvSmem);
    if (e != hipSuccess) return e;
    done.fetch_or(bit, std::memory_order_acq_rel);
  }
  return hipSuccess;
}

template <int T, int RT, bool XBF16, bool DQ, bool PAIR>
hipError_t launch_t(const GemvArgs& a, int grid_x, hipStream_t stream) {
  auto* fn = &gemv_splitk_kernel<T, RT, XBF16, DQ, PAIR>;
  hipError_t e = ensure_lds_attribute(fn);
  if (e != hipSuccess) return e;
  fn<<<dim3(grid_x, a.splits), kThreads, kGemvSmem, stream>>>(a);
  return hipGetLastError();
}

template <int T, int RT, bool PAIR>
hipError_t dispatch_flags(const GemvArgs& a, int grid_x, bool xbf16, bool dq, hipStream_t stream) {
  if (xbf16) return dq ? launch_t<T, RT, true, true, PAIR>(a, grid_x, stream)
                       : launch_t<T, RT, true, false, PAIR>(a, grid_x, stream);
  return dq ? launch_t<T, RT, false, true, PAIR>(a, grid_x, stream)
            : launch_t<T, RT, false, false, PAIR>(a, grid_x, stream);
}

// Instantiated (T, RT, PAIR) combinations; RT is the plan's rows per thread.
template <int T, bool PAIR>
hipError_t dispatch_rt(const GemvArgs& a, int grid_x, int rt, bool xbf16, bool dq, hipStream_t stream) {
  if constexpr (T == 1 && !PAIR) {
    if (rt == 16) return dispatch_flags<T, 16, PAIR>(a, grid_x, xbf16, dq, stream);
  }
  if constexpr (T <= 2 && !PAIR) {
    if (rt == 8) return dispatch_flags<T, 8, PAIR>(a, grid_x, xbf16, dq, stream);
  }
  if constexpr (!(PAIR && T > 1)) {
    if (rt == 4) return dispatch_flags<T, 4, PAIR>(a, grid_x, xbf16, dq, stream);
  }
  if constexpr (T == 1) {
    if (rt == 1) return dispatch_flags<T, 1, PAIR>(a, grid_x, xbf16, dq, stream);
  }
  return dispatch_flags<T, 2, PAIR>(a, grid_x, xbf16, dq, stream);
}

int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace

GemvPlan plan_gemv(int rows, int d_in, const int* d_out, int nweights, bool pair) {
  GemvPlan p{};
  p.pair = pair;
  int tiles = 0;
  const int nw_tiles = pair ? 1 : nweights;
  for (int i = 0; i < nw_tiles; ++i) tiles += ceil_div(d_out[i], kTileCols);
  // Split-K: about one workgroup per CU (256), since every workgroup pays a
  // fixed LUT build, reduction and hand-off; slabs of at least one 64-row
  // step and at most the rows per thread the register budget allows (16 for
  // one activation row, 8 for two, 4 beyond or in PAIR mode, 2 for a PAIR of
  // two).
  const int cap = pair ? (rows <= 1 ? 4 : 2) : (rows <= 1 ? 16 : (rows == 2 ? 8 : 4));
  int splits = 256 / tiles > 1 ? 256 / tiles : 1;
  if (splits > ceil_div(d_in, kRowGroups)) splits = ceil_div(d_in, kRowGroups);
  int rows_per_wg = ceil_div(d_in, splits);
  if (rows_per_wg > kRowGroups * cap) rows_per_wg = kRowGroups * cap;
  splits = ceil_div(d_in, rows_per_wg);
  int rt = 1;
  while (rt * kRowGroups < rows_per_wg) rt *= 2;
  p.rows_per_thread = rt;
  p.rows_per_wg = rows_per_wg;
  p.splits = splits;
  p.tiles = tiles;
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
  const int grid_x = t;
  const bool dq = weights[0].scales.kind == kScalesDQ;
  const int rt = p.rows_per_thread;
  if (p.pair) {
    if (rows == 1) return dispatch_rt<1, true>(a, grid_x, rt, x_bf16, dq, stream);
    if (rows == 2) return dispatch_rt<2, true>(a, grid_x, rt, x_bf16, dq, stream);
    return hipErrorInvalidValue;
  }
  switch (rows) {
    case 1: return dispatch_rt<1, false>(a, grid_x, rt, x_bf16, dq, stream);
    case 2: return dispatch_rt<2, false>(a, grid_x, rt, x_bf16, dq, stream);
    case 3: return dispatch_rt<3, false>(a, grid_x, rt, x_bf16, dq, stream);
    case 4: return dispatch_rt<4, false>(a, grid_x, rt, x_bf16, dq, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace unifur
