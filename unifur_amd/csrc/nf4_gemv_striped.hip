// nf4_gemv_striped.hip -- decode GEMV over the column-striped weight layout.
//
// y[t][o] = sum_i x[t][i] * deq(W)[i][o] (+ bias[o]) (+ LoRA), W an NF4
// weight [d_in = K, d_out = N] stored striped (nf4_layout.hip): 16-column
// stripe s holds K rows of 8 code bytes back to back, scales are [N/64][K].
// This is Nf4Linear::forward (src/qwennet.rs:238-241, dequantize then
// linear) and QloraLinear::forward (src/qwennet.rs:325-345) for a few rows
// of x, without materialising the weight.
//
// One workgroup owns one stripe over all of K, so there is no cross-workgroup
// reduction: its W waves take consecutive row ranges, and inside a wave lane
// l takes rows RPL (64 c + l) .. + RPL - 1 of every 64 RPL-row chunk c (RPL =
// 2 for the single-weight and shared-input launches, 1 for the SwiGLU pair)
// -- a wave's load of a chunk is 512 RPL contiguous bytes of codes, 64 RPL
// contiguous scale codes and 64 RPL contiguous activations per x row.  Each
// wave keeps D chunks in flight in a register
// ring: chunk c + D is requested as soon as chunk c has been consumed, so the
// memory stream and the decode overlap.  (Requesting everything up front
// stalls the issue of the later loads behind the memory system, and the
// decode then starts only once most data has arrived.)
//
// Decode: a byte of codes is looked up in a 256-entry LDS table holding
// {level[lo], level[hi]} (16 copies, lane l reads copy l % 16, so the 64-bit
// reads of 16 lanes hit distinct bank pairs; 32 KiB, so four workgroups fit
// a CU); the address is one v_perm_b32 (byte << 8 | lane offset) and a shift.  Per row and 64-block the activation is folded
// with the block scale once (xs = x * scale), then one FMA per code.  The
// lookups of chunk c + 1 are issued before the FMAs of chunk c.
//
// Reduction: the 16 column sums of each lane are added over the 64 lanes by
// a butterfly that halves the live columns at each step (permlane32 and
// permlane16 swaps, then row_mirror and row_half_mirror DPP), so every lane
// ends with one column; the W waves are then added through LDS in a fixed
// order.  Results are deterministic run to run.
//
// PAIR mode computes gate and up of a SwiGLU block in the same pass over x
// and stores silu(gate x) * (up x) (src/qwennet.rs:816-819,
// src/tensor_ext.rs:87-90).
#include "nf4_gemv.hpp"
#include "nf4_layout.hpp"

#include <atomic>
#include <type_traits>

namespace unifur {
namespace {

#ifndef UNIFUR_GEMV_LUT_COPIES
#define UNIFUR_GEMV_LUT_COPIES 16
#endif
constexpr int kLutCopies = UNIFUR_GEMV_LUT_COPIES;
static_assert(kLutCopies == 8 || kLutCopies == 16 || kLutCopies == 32, "LUT copies");
constexpr int kLutBytes = 256 * kLutCopies * 8;  // at LDS address 0
constexpr int kDqLutOffset = kLutBytes;          // one 256-entry DQ scale table per weight
constexpr int kStripedSmem = kDqLutOffset + 2 * 256 * 4;
// the GEMV's reduction space after the LUTs: (NW * T * W * 16 + T * W)
// floats, at most 2 * 2 * 8 * 16 + 64 (pair), 4 * 8 * 16 + 32, 2 * 16 * 16 + 32
constexpr int kGemvRedOffset = kStripedSmem;
constexpr int kGemvSmem = kGemvRedOffset + (512 + 64) * 4;

typedef __attribute__((address_space(3))) const f32x2 lds_f32x2;

__device__ __forceinline__ float as_f(uint32_t u) { return __uint_as_float(u); }

// NF4_LEVELS[c] for a per-lane c from immediates (no memory access).
__device__ __forceinline__ float level_select(int c) {
  float v = __uint_as_float(level_bits(0));
#pragma unroll
  for (int i = 1; i < 16; ++i) v = c == i ? __uint_as_float(level_bits(i)) : v;
  return v;
}
__device__ __forceinline__ uint32_t as_u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float silu_f32(float z) { return z * (1.0f / (1.0f + __expf(-z))); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Workgroup index in XCD-aware order: blockIdx.x % 8 is the XCD it runs on,
// and with run = gridDim.x / 8 (0 when 8 does not divide the grid) XCD x
// takes the run of indices from x * run.  A select, not a branch, so that
// the argument loads after it are not held behind the load of run.
__device__ __forceinline__ int xcd_order(int run) {
  const uint32_t bid = blockIdx.x;
  const uint32_t r = (bid & 7u) * (uint32_t)run + (bid >> 3);
  return (int)__builtin_amdgcn_readfirstlane(run != 0 ? r : bid);
}

// What the first loads of weight slot wi need -- its first stripe, codes,
// block scales and scale of scales -- read from every slot at fixed offsets
// and picked by wi: indexed by wi, these argument loads waited for the ones
// wi is found from, a second round trip before any weight byte is requested.
struct SlotHead {
  int stripe_begin;
  const uint8_t* packed;
  const void* scales;  // u8 DQ codes or f32 absmax
  const float* scale_of_scales;
};
__device__ __forceinline__ SlotHead slot_read(const StripedArgs& a, int i) {
  SlotHead c{a.stripe_begin[i], a.slot[i].packed, a.slot[i].scales, a.slot[i].scale_of_scales};
  // an empty operand barrier (no instruction): the values are loaded here,
  // so the selection below cannot become a load through a selected address
  asm volatile("" : "+s"(c.stripe_begin), "+s"(c.packed), "+s"(c.scales), "+s"(c.scale_of_scales));
  return c;
}
__device__ __forceinline__ SlotHead slot_head(const StripedArgs& a, int wi) {
  SlotHead h = slot_read(a, 0);
#pragma unroll
  for (int i = 1; i < kMaxGemvWeights; ++i) {
    const SlotHead c = slot_read(a, i);
    if (wi == i) h = c;
  }
  return h;
}

// The slot records of a launch's weights (the rest stay zero).
void set_slots(StripedArgs& a, const GemvWeight* weights, int nweights) {
  for (int i = 0; i < nweights; ++i) {
    const ScalesArg& sc = weights[i].scales;
    a.slot[i] = StripedSlot{weights[i].packed,
                            sc.kind == kScalesDQ ? static_cast<const void*>(sc.dq_codes)
                                                 : static_cast<const void*>(sc.absmax),
                            sc.scale_of_scales};
  }
}

// The scale of scales of a double-quantized weight as a vector load (every
// lane reads the one float), issued ahead of a launch's first chunk loads:
// vector loads return in order, so the first chunk's wait covers it.  Read
// through the scalar cache instead it held the LUT barrier, which waits on
// the LDS stores with the one counter that scalar loads share, until the
// value arrived behind every workgroup's first chunks.
__device__ __forceinline__ float load_scale_of_scales(const float* p) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(make_rsrc(p, 4u), 0, 0, 0));
}

// One chunk of one weight in flight: this lane's code bytes (8 per row) and
// row scales, for RPL consecutive rows per lane (a chunk is 64 RPL rows).
// Narrow loads are kept in narrow fields: the ring is carried around the
// chunk loop, and a widening of a loaded byte placed at the loop head would
// wait there for the newest loads instead of the ones the step consumes.
template <bool DQ, int RPL>
struct ChunkW {
  std::conditional_t<RPL == 1, u32x2, u32x4> code;
  // u8 DQ scale codes (RPL of them), or f32 absmax bits
  std::conditional_t<DQ, std::conditional_t<RPL == 1, uint8_t, uint16_t>, std::conditional_t<RPL == 1, uint32_t, u32x2>>
      scale;
};

template <int T, int NW, bool XBF16, bool DQ, int RPL>
struct Chunk {
  ChunkW<DQ, RPL> w[NW];
  // x of the RPL rows: bf16 or f32 bits
  std::conditional_t<XBF16, std::conditional_t<RPL == 1, uint16_t, uint32_t>, std::conditional_t<RPL == 1, uint32_t, u32x2>>
      x[T];
  std::conditional_t<RPL == 1, uint32_t, u32x2> g;  // with a folded norm: the rows' norm weights (f32 bits)
};

// Field accessors by row r < RPL of the lane.
template <bool DQ, int RPL>
__device__ __forceinline__ uint32_t code_dword(const ChunkW<DQ, RPL>& c, int r, int d) {
  return c.code[2 * r + d];
}
template <bool DQ, int RPL>
__device__ __forceinline__ uint32_t scale_bits(const ChunkW<DQ, RPL>& c, int r) {
  if constexpr (RPL == 1) return (uint32_t)c.scale;
  else if constexpr (DQ) return ((uint32_t)c.scale >> (8 * r)) & 0xffu;
  else return c.scale[r];
}
template <bool XBF16, typename X>
__device__ __forceinline__ float x_value(const X& v, int r) {
  if constexpr (std::is_same_v<X, uint16_t>) return bf16_bits_to_f32((uint32_t)v);
  else if constexpr (std::is_same_v<X, uint32_t>) return XBF16 ? bf16_bits_to_f32((v >> (16 * r)) & 0xffffu) : __uint_as_float(v);
  else return __uint_as_float(v[r]);
}
template <typename G>
__device__ __forceinline__ float g_value(const G& v, int r) {
  if constexpr (std::is_same_v<G, uint32_t>) return __uint_as_float(v);
  else return __uint_as_float(v[r]);
}

// Wave-uniform resources of one weight, bounded to this wave's rows so that
// every load past them reads zero (and touches no memory).
struct WaveW {
  __amdgpu_buffer_rsrc_t codes, scales;
};

template <int T, int NW, bool XBF16, bool DQ, bool NORM, int RPL>
__device__ __forceinline__ void issue_chunk(Chunk<T, NW, XBF16, DQ, RPL>& c, const WaveW (&ww)[NW],
                                            const __amdgpu_buffer_rsrc_t (&xr)[T], __amdgpu_buffer_rsrc_t gr,
                                            int chunk, int lane) {
  const uint32_t row = (uint32_t)((chunk * 64 + lane) * RPL);  // the lane's first row
  if constexpr (NORM) {  // 0 without a norm
    if constexpr (RPL == 1) c.g = __builtin_amdgcn_raw_buffer_load_b32(gr, row * 4u, 0, 0);
    else c.g = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(gr, row * 4u, 0, 0));
  }
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    if constexpr (RPL == 1)
      c.w[w].code = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(ww[w].codes, row * 8u, 0, 0));
    else
      c.w[w].code = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ww[w].codes, row * 8u, 0, 0));
    if constexpr (DQ && RPL == 1)
      c.w[w].scale = __builtin_amdgcn_raw_buffer_load_b8(ww[w].scales, row, 0, 0);
    else if constexpr (DQ)
      c.w[w].scale = __builtin_amdgcn_raw_buffer_load_b16(ww[w].scales, row, 0, 0);
    else if constexpr (RPL == 1)
      c.w[w].scale = __builtin_amdgcn_raw_buffer_load_b32(ww[w].scales, row * 4u, 0, 0);
    else
      c.w[w].scale = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(ww[w].scales, row * 4u, 0, 0));
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if constexpr (XBF16 && RPL == 1)
      c.x[t] = __builtin_amdgcn_raw_buffer_load_b16(xr[t], row * 2u, 0, 0);
    else if constexpr (XBF16)
      c.x[t] = __builtin_amdgcn_raw_buffer_load_b32(xr[t], row * 2u, 0, 0);
    else if constexpr (RPL == 1)
      c.x[t] = __builtin_amdgcn_raw_buffer_load_b32(xr[t], row * 4u, 0, 0);
    else
      c.x[t] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(xr[t], row * 4u, 0, 0));
  }
}

// Level pairs of this lane's code bytes and its row scales, per weight.
template <int NW, int RPL>
struct Looked {
  f32x2 lv[NW][8 * RPL];
  float scale[NW][RPL];
};

template <int T, int NW, bool XBF16, bool DQ, int RPL>
__device__ __forceinline__ void lookup(Looked<NW, RPL>& o, const Chunk<T, NW, XBF16, DQ, RPL>& c, const float* dq_lut,
                                       const float (&sos)[NW], uint32_t lane_off) {
  // lane_off is (copy * 8) << (8 - log2(kLutCopies * 8 / 32)): the v_perm
  // puts the code byte in bits 8-15, and a shift brings the entry stride down
  // to kLutCopies * 8 bytes when that is under 256.
  constexpr int kShift = kLutCopies == 32 ? 0 : (kLutCopies == 16 ? 1 : 2);
#pragma unroll
  for (int w = 0; w < NW; ++w) {
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      // DQ: ((float)q / 255.0f) * scale_of_scales (src/quantize.rs:349), the
      // quotient from the table and the product here (the same two roundings)
      const uint32_t sb = scale_bits<DQ, RPL>(c.w[w], r);
      o.scale[w][r] = DQ ? dq_lut[sb] * sos[w] : as_f(sb);
#pragma unroll
      for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          // LDS byte address = (byte b of the dword) << 8 | lane_off; the LUT
          // sits at LDS address 0 (this kernel has no static LDS)
          const uint32_t addr =
              perm_b32(code_dword<DQ, RPL>(c.w[w], r, d), lane_off, 0x0c0c0000u | ((4u + b) << 8)) >> kShift;
          o.lv[w][r * 8 + d * 4 + b] = *reinterpret_cast<lds_f32x2*>((size_t)addr);
        }
    }
  }
}

// Sum v[16] over the 64 lanes; lane l ends with column ci(l) (see below) in
// its return value (lanes l, l^1, l^2, l^3 hold the same column).
__device__ __forceinline__ float wave_column_sum(const float (&acc)[16], int lane) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // lane bit 5: lanes 0-31 keep columns 0-7, 32-63 keep 8-15
    auto r = __builtin_amdgcn_permlane32_swap(as_u(acc[i]), as_u(acc[i + 8]), false, false);
    v[i] = as_f(r[0]) + as_f(r[1]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // lane bit 4 (odd rows of 16 keep the upper half)
    auto r = __builtin_amdgcn_permlane16_swap(as_u(v[i]), as_u(v[i + 4]), false, false);
    v[i] = as_f(r[0]) + as_f(r[1]);
  }
  {  // lane bit 3: partner 15 - l within the row (row_mirror)
    const bool hi = (lane & 8) != 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float send = hi ? v[i] : v[i + 2];
      const float keep = hi ? v[i + 2] : v[i];
      v[i] = keep + as_f(dpp_mov<0x140>(as_u(send)));
    }
  }
  float col;
  {  // lane bit 2: partner 7 - l within the half row (row_half_mirror)
    const bool hi = (lane & 4) != 0;
    const float send = hi ? v[0] : v[1];
    const float keep = hi ? v[1] : v[0];
    col = keep + as_f(dpp_mov<0x141>(as_u(send)));
  }
  // the four lanes of a quad now hold the same column: add them
  col += as_f(dpp_mov<0x4E>(as_u(col)));  // quad_perm [2,3,0,1]
  col += as_f(dpp_mov<0xB1>(as_u(col)));  // quad_perm [1,0,3,2]
  return col;
}

__device__ __forceinline__ int wave_column_index(int lane) {
  return ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1);
}

// Sum of v over the 64 lanes, in every lane.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
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

// y (+ residual[idx], the residual stream a decoder layer adds its
// projection to: src/qwennet.rs:1124-1128), stored in y's dtype.
__device__ __forceinline__ void store_y(const GemvWeight& W, size_t idx, float y) {
  if (W.residual)
    y += W.y_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(W.residual)[idx])
                  : reinterpret_cast<const float*>(W.residual)[idx];
  if (W.y_bf16)
    reinterpret_cast<uint16_t*>(W.y)[idx] = (uint16_t)(pack_bf16x2(y, 0.0f) & 0xffffu);
  else
    reinterpret_cast<float*>(W.y)[idx] = y;
}

// What the prologue of a one-weight launch reads comes first, as scalar
// parameters: the build preloads the leading kernel arguments into SGPRs
// (amdgpu-kernarg-preload-count), so those need no load through the scalar
// cache before the first weight byte is requested.  x_arg, slot0, d_in,
// rows_per_wave, xcd_run and nweights repeat the fields of a; a launch with
// several weights (or the SwiGLU pair) reads the other slots from a.
template <int T, int W, int D, bool XBF16, bool DQ, bool PAIR, bool NORM, int RPL>
__global__ __launch_bounds__(W * 64) void gemv_striped_kernel(const void* x_arg, const uint8_t* packed0,
                                                              const void* scales0, const float* sos0, int d_in_arg,
                                                              int rows_per_wave_arg, int xcd_run_arg,
                                                              int nweights_arg, StripedArgs a) {
  constexpr int NW = PAIR ? 2 : 1;
  static_assert(RPL == 1 || RPL == 2, "one or two rows per lane and chunk");
  static_assert(D % 2 == 0, "the lookup double buffer is indexed by chunk parity");
  static_assert(W >= 4, "the LUT build needs 256 threads");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // XCD-aware order: workgroup b runs on XCD b % 8, so each XCD takes a
  // contiguous run of stripes and the four stripes of a 64-column block
  // (which share their scale codes) meet in one L2.  The run length comes
  // with the arguments: derived from gridDim here, it put a load of the grid
  // size and a branch ahead of every other argument load.
  const int b = xcd_order(xcd_run_arg);
  // which weight (several weights of one x can share a launch) and stripe
  int wi = 0;
  SlotHead head[NW];
  head[0] = SlotHead{0, packed0, scales0, sos0};  // slot 0 starts at stripe 0
  if constexpr (PAIR) {
    head[1] = slot_read(a, 1);
  } else if (nweights_arg > 1) {
#pragma unroll
    for (int i = 1; i < kMaxGemvWeights; ++i)
      if (i < nweights_arg && b >= a.stripe_begin[i]) wi = i;
    head[0] = slot_head(a, wi);
  }
  const int s = b - head[0].stripe_begin;
  const int K = d_in_arg;
  const int kw = wave * rows_per_wave_arg;
  const int nrows = max(0, min(rows_per_wave_arg, K - kw));
  const int nchunks = (nrows + 64 * RPL - 1) / (64 * RPL);

  WaveW ww[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    ww[w].codes = make_rsrc(head[w].packed + ((size_t)s * K + kw) * 8, (uint32_t)nrows * 8u);
    const size_t srow = (size_t)(s / 4) * K + kw;
    ww[w].scales = DQ ? make_rsrc(static_cast<const uint8_t*>(head[w].scales) + srow, (uint32_t)nrows)
                      : make_rsrc(static_cast<const float*>(head[w].scales) + srow, (uint32_t)nrows * 4u);
  }
  __amdgpu_buffer_rsrc_t xr[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const size_t off = (size_t)t * K + kw;
    xr[t] = XBF16 ? make_rsrc(static_cast<const uint16_t*>(x_arg) + off, (uint32_t)nrows * 2u)
                  : make_rsrc(static_cast<const float*>(x_arg) + off, (uint32_t)nrows * 4u);
  }
  // folded QwenRmsNorm (src/qwennet.rs:104-109): the products take
  // x * (w + 1), each lane sums x^2 over its rows, and the column sums are
  // scaled by the row's 1 / sqrt(mean(x^2) + eps) at the end.  NORM kernels
  // do this work in every chunk; one launched without a norm gets a weight
  // buffer with no records, whose loads read 0, so x is multiplied by exactly
  // 1 -- the loop has no branch on the norm (a branch there made the
  // compiler keep two versions of the loop and double the registers).  The
  // single-weight kernels come in both forms (the norm weight's load is a
  // quarter of a chunk's loads: config 2 9.0 -> 8.5 us without it); the
  // SwiGLU pair keeps one, which measured faster with the loads than without.
  const bool norm = NORM && a.norm_w != nullptr;
  const __amdgpu_buffer_rsrc_t gr = make_rsrc(norm ? a.norm_w + kw : x_arg, norm ? (uint32_t)nrows * 4u : 0u);

  // The prologue issues the first D chunks, in chunk order like the steady
  // state (a load of chunk 0 issued last would make every pass through the
  // loop head wait for the newest loads), before the LUT build, so that
  // their memory latency overlaps the build and its barrier (config 2:
  // 8.85 -> 8.65 us per launch).  The DQ table holds q / 255 and the scale
  // of scales, loaded ahead of the chunks, is applied per row, so the table
  // does not wait for that load.
  float sos[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w)
    sos[w] = DQ ? load_scale_of_scales(head[w].scale_of_scales) : 1.0f;
  __builtin_amdgcn_sched_barrier(0);
  Chunk<T, NW, XBF16, DQ, RPL> ring[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    issue_chunk<T, NW, XBF16, DQ, NORM, RPL>(ring[j], ww, xr, gr, j, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (tid < 256) {
    const float lo = level_select(tid & 15), hi = level_select(tid >> 4);
    const f32x4 v = {lo, hi, lo, hi};
    f32x4* dst = reinterpret_cast<f32x4*>(smem + tid * (kLutCopies * 8));
#pragma unroll
    for (int j = 0; j < kLutCopies / 2; ++j) dst[(j + tid) & (kLutCopies / 2 - 1)] = v;
    if constexpr (DQ) reinterpret_cast<float*>(smem + kDqLutOffset)[tid] = (float)tid / 255.0f;
  }
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);

  const float* dq_lut = reinterpret_cast<const float*>(smem + kDqLutOffset);
  const uint32_t lane_off = ((uint32_t)(lane & (kLutCopies - 1)) * 8u) << (kLutCopies == 32 ? 0 : kLutCopies == 16 ? 1 : 2);
  float acc[NW][T][16];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[w][t][i] = 0.0f;
  float xsq[T];
#pragma unroll
  for (int t = 0; t < T; ++t) xsq[t] = 0.0f;

  Looked<NW, RPL> lk[2];
  lookup<T, NW, XBF16, DQ, RPL>(lk[0], ring[0], dq_lut, sos, lane_off);
  for (int c0 = 0; c0 < nchunks; c0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      // chunk c0 + j is in ring[j] and already looked up in lk[j & 1];
      // chunk c0 + j + 1 is in ring[(j + 1) % D] (refilled at step 0 when
      // j + 1 == D).  Chunks past this wave's rows read as zero: x = 0.
      __builtin_amdgcn_sched_barrier(0);
      lookup<T, NW, XBF16, DQ, RPL>(lk[(j + 1) & 1], ring[(j + 1) % D], dq_lut, sos, lane_off);
      float xs[NW][T][RPL];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
          float xv = x_value<XBF16>(ring[j].x[t], r);
          if constexpr (NORM) {
            xsq[t] = __builtin_fmaf(xv, xv, xsq[t]);
            xv = xv * (g_value(ring[j].g, r) + 1.0f);
          }
#pragma unroll
          for (int w = 0; w < NW; ++w) xs[w][t][r] = xv * lk[j & 1].scale[w][r];  // x * block scale, once per row
        }
      issue_chunk<T, NW, XBF16, DQ, NORM, RPL>(ring[j], ww, xr, gr, c0 + j + D, lane);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int r = 0; r < RPL; ++r)
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int t = 0; t < T; ++t) {
              acc[w][t][2 * i] = __builtin_fmaf(xs[w][t][r], lk[j & 1].lv[w][r * 8 + i].x, acc[w][t][2 * i]);
              acc[w][t][2 * i + 1] = __builtin_fmaf(xs[w][t][r], lk[j & 1].lv[w][r * 8 + i].y, acc[w][t][2 * i + 1]);
            }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // reduce: over the lanes of each wave, then over the waves (LUT space reused)
  float col[NW][T];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int t = 0; t < T; ++t) col[w][t] = wave_column_sum(acc[w][t], lane);
  float* red = reinterpret_cast<float*>(smem + kGemvRedOffset);  // past the LUTs: no barrier before writing it
  if ((lane & 3) == 0) {
    const int ci = wave_column_index(lane);
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int t = 0; t < T; ++t) red[((w * T + t) * W + wave) * 16 + ci] = col[w][t];
  }
  float* red_sq = red + NW * T * W * 16;  // the waves' sums of x^2, per row
  if (norm) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float v = wave_sum(xsq[t]);
      if (lane == 0) red_sq[t * W + wave] = v;
    }
  }
  __syncthreads();
  if (tid >= T * 16) return;
  const int t = tid / 16, cc = tid % 16;
  const GemvWeight& G = a.w[wi];
  const int gcol = s * kStripeCols + cc;
  float sum[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    float v = 0.0f;
#pragma unroll
    for (int q = 0; q < W; ++q) v += red[((w * T + t) * W + q) * 16 + cc];
    sum[w] = v;
  }
  if (norm) {
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < W; ++q) ss += red_sq[t * W + q];
    // (mean(x^2) + eps)^(-1/2), the factor every normed x of this row carries
    const float inv = 1.0f / __builtin_sqrtf(ss / (float)K + a.norm_eps);
#pragma unroll
    for (int w = 0; w < NW; ++w) sum[w] *= inv;
  }
  float y = epilogue_value(G, sum[0], t, gcol);
  if constexpr (PAIR) y = silu_f32(y) * epilogue_value(a.w[1], sum[1], t, gcol);  // silu(gate x) * up x
  store_y(G, (size_t)t * G.d_out + gcol, y);
}

// ================================================================ launching ==

#ifndef UNIFUR_GEMV_DEPTH
#define UNIFUR_GEMV_DEPTH 4
#endif
constexpr int kDepth = UNIFUR_GEMV_DEPTH;
// rows per lane of the single-weight and shared-input kernels, and their
// ring depth: two rows per lane (one 16-byte code load, paired scale and x
// loads: half the load instructions) with two chunks in flight -- the same
// bytes in flight as four one-row chunks -- measured config 2 8.59 -> 8.33
// us; four two-row chunks in flight 9.05 us
#ifndef UNIFUR_GEMV_RPL
#define UNIFUR_GEMV_RPL 2
#endif
#ifndef UNIFUR_GEMV_DEPTH2
#define UNIFUR_GEMV_DEPTH2 2
#endif
constexpr int kRpl = UNIFUR_GEMV_RPL;

template <bool PAIR>
constexpr int NWof() { return PAIR ? 2 : 1; }

template <int T, int W, bool XBF16, bool DQ, bool PAIR, bool NORM, int RPL = 1>
hipError_t launch_t(const StripedArgs& a, int grid, hipStream_t stream) {
  auto* fn = &gemv_striped_kernel<T, W, RPL == 1 ? kDepth : UNIFUR_GEMV_DEPTH2, XBF16, DQ, PAIR, NORM, RPL>;
  static std::atomic<uint64_t> done{0};  // dynamic LDS above 64 KiB: once per device
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(done.load(std::memory_order_acquire) & bit)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kGemvSmem);
    if (e != hipSuccess) return e;
    done.fetch_or(bit, std::memory_order_acq_rel);
  }
  static_assert(NWof<PAIR>() * T * W * 16 + T * W <= 512 + 64, "GEMV reduction space");
  StripedArgs args = a;
  args.xcd_run = grid % 8 == 0 ? grid / 8 : 0;
  fn<<<grid, W * 64, kGemvSmem, stream>>>(args.x, args.slot[0].packed, args.slot[0].scales,
                                          args.slot[0].scale_of_scales, args.d_in, args.rows_per_wave, args.xcd_run,
                                          args.nweights, args);
  return hipGetLastError();
}

template <int T, int W, bool PAIR, bool NORM>
hipError_t launch_norm(const StripedArgs& a, int grid, bool xbf16, bool dq, hipStream_t stream) {
  if constexpr (kRpl == 2 && !PAIR) {
    // two rows per lane: even d_in (a lane's rows are both in or both past
    // its wave's rows), x and the norm weight aligned for the paired loads
    const size_t xa = xbf16 ? 4 : 8;
    if (a.d_in % 2 == 0 && reinterpret_cast<uintptr_t>(a.x) % xa == 0 &&
        reinterpret_cast<uintptr_t>(a.norm_w) % 8 == 0) {
      if (xbf16)
        return dq ? launch_t<T, W, true, true, PAIR, NORM, 2>(a, grid, stream)
                  : launch_t<T, W, true, false, PAIR, NORM, 2>(a, grid, stream);
      return dq ? launch_t<T, W, false, true, PAIR, NORM, 2>(a, grid, stream)
                : launch_t<T, W, false, false, PAIR, NORM, 2>(a, grid, stream);
    }
  }
  if (xbf16)
    return dq ? launch_t<T, W, true, true, PAIR, NORM>(a, grid, stream) : launch_t<T, W, true, false, PAIR, NORM>(a, grid, stream);
  return dq ? launch_t<T, W, false, true, PAIR, NORM>(a, grid, stream) : launch_t<T, W, false, false, PAIR, NORM>(a, grid, stream);
}

// the SwiGLU pair always takes the NORM kernel (norm or not, see above)
template <int T, int W, bool PAIR>
hipError_t launch_flags(const StripedArgs& a, int grid, bool xbf16, bool dq, hipStream_t stream) {
  if (PAIR || a.norm_w) return launch_norm<T, W, PAIR, true>(a, grid, xbf16, dq, stream);
  return launch_norm<T, W, PAIR, false>(a, grid, xbf16, dq, stream);
}

// 16 waves only where the registers fit at four waves per SIMD: one or two
// activation rows of a single weight (the plan never asks for more).
template <int T, bool PAIR>
hipError_t dispatch_w(const StripedArgs& a, int grid, int waves, bool xbf16, bool dq, hipStream_t stream) {
  if (waves == 4) return launch_flags<T, 4, PAIR>(a, grid, xbf16, dq, stream);
  if (waves == 8) return launch_flags<T, 8, PAIR>(a, grid, xbf16, dq, stream);
  if constexpr (T <= 2 && !PAIR) {
    if (waves == 16) return launch_flags<T, 16, PAIR>(a, grid, xbf16, dq, stream);
  }
  return hipErrorInvalidValue;
}

// ============================================== 5..64 rows on MFMA (skinny) ==
//
// The GEMV's decomposition (waves split d_in, 64-row chunks, register ring)
// with the products on v_mfma_f32_16x16x32_bf16 (C[token][column] +=
// A[token][k] B[k][column]).  A wave owns S consecutive stripes (S = 1, 2 or
// 4, inside one 64-column block, so they share the row scales) of NW weights
// (2 for the SwiGLU gate/up pair): every activation load feeds NW * S
// stripes.  For each chunk and each (weight, stripe) unit:
//   * the wave writes the unit's 64 x 8 code bytes to a private LDS slot
//     (lane = row) and reads them back with ds_read_b64_tr_b4, which
//     transposes 16 x 16 nibbles inside each group of 16 lanes: lane 16 G + c
//     receives column c of rows 16 G .. 16 G + 15 -- the MFMA operand layout
//     (8 consecutive k per lane), rows 16 G + j, j < 8 for the first MFMA of
//     the chunk and j >= 8 for the second;
//   * each byte (two rows of one column) is looked up in the level-pair LUT,
//     multiplied by the two row scales -- the scale of row 16 G + j is decoded
//     by lane 16 G + j and broadcast with DPP row_newbcast:j -- and rounded to
//     a bf16 pair: the B operand is bf16(level * scale), what the MFMA GEMM
//     path stages in LDS;
//   * the A operand is x itself: lane 16 G + t holds x[t][k .. k + 15] of its
//     group's 16 rows (two 16-byte loads per 16-token tile, up to four
//     tiles); loads outside the wave's rows or past the tokens read zero.
// The units are software-pipelined: the LDS work of the next unit is issued
// before the MFMAs of the current one.  The waves' accumulators are added
// through LDS in a fixed order.

typedef int v2i32 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i32 lds_v2i32;

typedef __attribute__((address_space(3))) u32x2 lds_u32x2_w;

constexpr int kSkStageOffset = kStripedSmem;  // after the level and DQ LUTs

// the value of lane 16 (l / 16) + J, in every lane l
template <int J>
__device__ __forceinline__ float row_bcast(float v) {
  return as_f(dpp_mov<0x150 + J>(as_u(v)));
}
template <int J>
__device__ __forceinline__ void row_bcast_all(float v, float (&o)[16]) {
  o[J] = row_bcast<J>(v);
  if constexpr (J + 1 < 16) row_bcast_all<J + 1>(v, o);
}

template <int NT, int NW, int S, bool DQ, bool XF32>
struct SkChunk {
  u32x2 code[NW][S];
  std::conditional_t<DQ, uint8_t, uint32_t> scale[NW];  // narrow, as in the GEMV ring
  u32x4 x[NT][XF32 ? 4 : 2];  // 16 activations of one token: bf16, or f32
  uint32_t g;  // NORM kernels: the norm weight of this lane's row (f32 bits)
};

// Loads of chunk `chunk` of this wave: codes of row 64 chunk + lane of each
// stripe and its scale, and for each token tile x[t][k0 .. k0 + 15] with
// t = 16 tt + lane % 16, k0 = kw + 64 chunk + 16 (lane / 16).  The code and
// scale buffers end at the wave's last row (stripes before the last read the
// next rows of their stripe, which meet zero scales and zero activations);
// activation offsets past the wave's rows are sent out of the buffer (zero),
// tokens past `rows` fall out of it by themselves.
template <int NT, int NW, int S, bool DQ, bool XF32, bool NORM>
__device__ __forceinline__ void sk_issue(SkChunk<NT, NW, S, DQ, XF32>& c, const WaveW (&ww)[NW],
                                         __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t gr, int K, int kw, int kend,
                                         int chunk, int lane) {
  const uint32_t row = (uint32_t)(chunk * 64 + lane);
  if constexpr (NORM) c.g = __builtin_amdgcn_raw_buffer_load_b32(gr, row * 4u, 0, 0);
#pragma unroll
  for (int w = 0; w < NW; ++w) {
#pragma unroll
    for (int i = 0; i < S; ++i)
      c.code[w][i] = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(ww[w].codes, ((uint32_t)(i * K) + row) * 8u, 0, 0));
    if constexpr (DQ)
      c.scale[w] = __builtin_amdgcn_raw_buffer_load_b8(ww[w].scales, row, 0, 0);
    else
      c.scale[w] = __builtin_amdgcn_raw_buffer_load_b32(ww[w].scales, row * 4u, 0, 0);
  }
  const int k0 = kw + chunk * 64 + 16 * (lane >> 4);
  constexpr uint32_t kEl = XF32 ? 4u : 2u;  // bytes per activation
  constexpr int kPer = XF32 ? 4 : 8;        // activations per 16-byte load
  const uint32_t off = (uint32_t)((lane & 15) * K + k0) * kEl;
  const uint32_t out = 0x80000000u;  // beyond num_records: reads zero
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const uint32_t o = off + (uint32_t)(16 * tt * K) * kEl;
#pragma unroll
    for (int q = 0; q < (XF32 ? 4 : 2); ++q)
      c.x[tt][q] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, k0 + kPer * (q + 1) <= kend ? o + 16u * q : out, 0, 0));
  }
}

// One unit's code bytes: stage, transpose, look up (level pairs of rows
// 16 G + 2 m, 16 G + 2 m + 1 of this lane's column, m = 0..7).
__device__ __forceinline__ void sk_lookup(f32x2 (&lv)[8], u32x2 code, uint32_t stage, uint32_t lane_off) {
  constexpr int kShift = kLutCopies == 32 ? 0 : (kLutCopies == 16 ? 1 : 2);
  *reinterpret_cast<lds_u32x2_w*>((size_t)stage) = code;
  const v2i32 nib = __builtin_amdgcn_ds_read_tr4_b64_v2i32(reinterpret_cast<lds_v2i32*>((size_t)stage));
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t addr = perm_b32((uint32_t)nib[d], lane_off, 0x0c0c0000u | ((4u + b) << 8)) >> kShift;
      lv[d * 4 + b] = *reinterpret_cast<lds_f32x2*>((size_t)addr);
    }
}

template <int NT, int W, int D, int S, bool DQ, bool PAIR, bool XF32, bool NORM>
__global__ __launch_bounds__(W * 64) void skinny_kernel(const void* x_arg, const uint8_t* packed0,
                                                        const void* scales0, const float* sos0, int d_in_arg,
                                                        int rows_per_wave_arg, int rows_per_split_arg, int rows_arg,
                                                        int xcd_run_arg, int nweights_arg, int splits_arg,
                                                        const float* norm_w_arg,
                                                        StripedArgs a) {  // leading parameters as in the GEMV
  constexpr int NW = PAIR ? 2 : 1;
  constexpr int U = NW * S;  // units per chunk
  static_assert(D % 2 == 0, "the scale double buffer is indexed by chunk parity");
  static_assert(W >= 4, "the LUT build and the epilogue need 256 threads");
  static_assert(S == 1 || S == 2 || S == 4, "stripes per wave stay inside one 64-column block");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int b = xcd_order(xcd_run_arg);  // as in the GEMV
  const int gs = b * S;  // first stripe of this workgroup over the launch
  int wi = 0;
  SlotHead head[NW];  // as in the GEMV
  head[0] = SlotHead{0, packed0, scales0, sos0};
  if constexpr (PAIR) {
    head[1] = slot_read(a, 1);
  } else if (nweights_arg > 1) {
#pragma unroll
    for (int i = 1; i < kMaxGemvWeights; ++i)
      if (i < nweights_arg && gs >= a.stripe_begin[i]) wi = i;
    head[0] = slot_head(a, wi);
  }
  const int s0 = gs - head[0].stripe_begin;
  const int K = d_in_arg;
  const int P = splits_arg, p = blockIdx.y;  // d_in slabs (gridDim.y)
  const int kw = p * rows_per_split_arg + wave * rows_per_wave_arg;
  const int nrows = max(0, min(rows_per_wave_arg, K - kw));
  const int nchunks = (nrows + 63) / 64;

  WaveW ww[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    ww[w].codes = make_rsrc(head[w].packed + ((size_t)s0 * K + kw) * 8, (uint32_t)((S - 1) * K + nrows) * 8u);
    const size_t srow = (size_t)(s0 / 4) * K + kw;
    ww[w].scales = DQ ? make_rsrc(static_cast<const uint8_t*>(head[w].scales) + srow, (uint32_t)nrows)
                      : make_rsrc(static_cast<const float*>(head[w].scales) + srow, (uint32_t)nrows * 4u);
  }
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x_arg, (uint32_t)rows_arg * (uint32_t)K * (XF32 ? 4u : 2u));
  // NORM: QwenRmsNorm over x folded in (src/qwennet.rs:104-109), over the
  // whole of d_in in one workgroup (no d_in slabs): each row's (w + 1) rides
  // on its block scale -- B = level * (scale * (w + 1)) -- each lane sums x^2
  // of the activations it feeds the MFMAs, and the outputs of token t are
  // scaled by 1 / sqrt(mean(x_t^2) + eps) before the epilogue
  const __amdgpu_buffer_rsrc_t gr = make_rsrc(NORM ? norm_w_arg + kw : x_arg, NORM ? (uint32_t)nrows * 4u : 0u);

  // as in the GEMV: the scale of scales and then the first chunks in flight
  // before the LUT build, the scale of scales applied per row (the DQ table
  // holds q / 255)
  float sos[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w)
    sos[w] = DQ ? load_scale_of_scales(head[w].scale_of_scales) : 1.0f;
  __builtin_amdgcn_sched_barrier(0);
  SkChunk<NT, NW, S, DQ, XF32> ring[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {  // in chunk order, as in the GEMV
    sk_issue<NT, NW, S, DQ, XF32, NORM>(ring[j], ww, xr, gr, K, kw, kw + nrows, j, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (tid < 256) {  // level-pair LUT and DQ scale table, as in the GEMV
    const float lo = level_select(tid & 15), hi = level_select(tid >> 4);
    const f32x4 v = {lo, hi, lo, hi};
    f32x4* dst = reinterpret_cast<f32x4*>(smem + tid * (kLutCopies * 8));
#pragma unroll
    for (int j = 0; j < kLutCopies / 2; ++j) dst[(j + tid) & (kLutCopies / 2 - 1)] = v;
    if constexpr (DQ) reinterpret_cast<float*>(smem + kDqLutOffset)[tid] = (float)tid / 255.0f;
  }
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);

  const float* dq_lut = reinterpret_cast<const float*>(smem + kDqLutOffset);
  const uint32_t lane_off = ((uint32_t)(lane & (kLutCopies - 1)) * 8u)
                            << (kLutCopies == 32 ? 0 : kLutCopies == 16 ? 1 : 2);
  const uint32_t stage = (uint32_t)(kSkStageOffset + wave * 512 + lane * 8);
  f32x4 acc[NW][S][NT];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int i = 0; i < S; ++i)
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) acc[w][i][tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float xsq[NT];  // NORM: this lane's sum of x^2 (token lane % 16 of each tile)
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) xsq[tt] = 0.0f;

  auto decode_scale = [&](const SkChunk<NT, NW, S, DQ, XF32>& c, int w) {
    // ((float)q / 255.0f) * scale_of_scales (src/quantize.rs:349)
    const float sc = DQ ? dq_lut[(uint32_t)c.scale[w]] * sos[w] : as_f((uint32_t)c.scale[w]);
    return NORM ? sc * (as_f(c.g) + 1.0f) : sc;  // NORM: the row's (w + 1) with its scale
  };
  float sdec[2][NW];  // this lane's row scale, per chunk parity
  f32x2 lk[2][8];     // level pairs, per unit parity
#pragma unroll
  for (int w = 0; w < NW; ++w) sdec[0][w] = decode_scale(ring[0], w);
  sk_lookup(lk[0], ring[0].code[0][0], stage, lane_off);
  for (int c0 = 0; c0 < nchunks; c0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      float sc[NW][16];
#pragma unroll
      for (int w = 0; w < NW; ++w) row_bcast_all<0>(sdec[j & 1][w], sc[w]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int w = u / S, i = u % S;
        const int q = j * U + u;  // unit parity (c0 * U is even)
        __builtin_amdgcn_sched_barrier(0);
        if (u + 1 < U) {
          sk_lookup(lk[(q + 1) & 1], ring[j].code[(u + 1) / S][(u + 1) % S], stage, lane_off);
        } else {
#pragma unroll
          for (int v = 0; v < NW; ++v) sdec[(j + 1) & 1][v] = decode_scale(ring[(j + 1) % D], v);
          sk_lookup(lk[(q + 1) & 1], ring[(j + 1) % D].code[0][0], stage, lane_off);
        }
        const f32x2(&L)[8] = lk[q & 1];
        if constexpr (XF32) {
          // f32 operands: B = level * scale exactly as the reference's
          // dequantized f32 value (src/quantize.rs:362), 16 MFMAs of 4 k
          // (lane group G supplies k = 16 G + m of MFMA m, for both operands)
#pragma unroll
          for (int m = 0; m < 16; ++m) {
            const float bm = ((m & 1) ? L[m >> 1].y : L[m >> 1].x) * sc[w][m];
#pragma unroll
            for (int tt = 0; tt < NT; ++tt)
              acc[w][i][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(as_f(ring[j].x[tt][m >> 2][m & 3]), bm,
                                                                   acc[w][i][tt], 0, 0, 0);
          }
        } else {
          u32x4 b0, b1;
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            b0[m] = pack_bf16x2(L[m].x * sc[w][2 * m], L[m].y * sc[w][2 * m + 1]);
            b1[m] = pack_bf16x2(L[4 + m].x * sc[w][8 + 2 * m], L[4 + m].y * sc[w][9 + 2 * m]);
          }
          const bf16x8_t B0 = __builtin_bit_cast(bf16x8_t, b0), B1 = __builtin_bit_cast(bf16x8_t, b1);
#pragma unroll
          for (int tt = 0; tt < NT; ++tt) {
            acc[w][i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ring[j].x[tt][0]),
                                                                    B0, acc[w][i][tt], 0, 0, 0);
            acc[w][i][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ring[j].x[tt][1]),
                                                                    B1, acc[w][i][tt], 0, 0, 0);
          }
        }
      }
      if constexpr (NORM) {  // x^2 of this chunk's activations, once per chunk
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
          for (int q = 0; q < (XF32 ? 4 : 2); ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t u = ring[j].x[tt][q][e];
              if constexpr (XF32) {
                xsq[tt] = __builtin_fmaf(as_f(u), as_f(u), xsq[tt]);
              } else {
                const float lo = as_f(u << 16), hi = as_f(u & 0xffff0000u);
                xsq[tt] = __builtin_fmaf(lo, lo, __builtin_fmaf(hi, hi, xsq[tt]));
              }
            }
      }
      sk_issue<NT, NW, S, DQ, XF32, NORM>(ring[j], ww, xr, gr, K, kw, kw + nrows, c0 + j + D, lane);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // NORM: the token sums of x^2 over the lane groups (lanes t, t + 16, t + 32,
  // t + 48 hold one token), then over the waves in wave order through LDS
  // (past the wave reduction's space, inside the LUT's), and each token's
  // 1 / sqrt(mean + eps) into LDS for the epilogue
  float* inv_tok = reinterpret_cast<float*>(smem + 16384) + NT * W * 16;
  if constexpr (NORM) {
    float* sq = reinterpret_cast<float*>(smem + 16384);
    float ss[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      float v = xsq[tt];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      ss[tt] = v;
    }
    __syncthreads();  // every wave is past its LUT lookups
    if (lane < 16) {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) sq[(tt * W + wave) * 16 + lane] = ss[tt];
    }
    __syncthreads();
    if (tid < NT * 16) {
      const int tt = tid >> 4, t = tid & 15;
      float v = 0.0f;
#pragma unroll
      for (int q = 0; q < W; ++q) v += sq[(tt * W + q) * 16 + t];
      inv_tok[tid] = 1.0f / __builtin_sqrtf(v / (float)K + a.norm_eps);
    }
  }

  // acc[w][i][tt][e] = C[token 16 tt + 4 (lane / 16) + e][column lane % 16 of
  // stripe s0 + i]; waves added through LDS (LUT space, below the norm's
  // sums at 16 KiB), both weights of a pair together, in wave order.  When
  // every (tile, stripe) fits there at once, one write phase and one read
  // phase (two barriers); else one (tile, stripe) at a time (two barriers
  // each).  Thread tid < 256 owns token 16 tt + tid / 16, column tid % 16 of
  // every (tile, stripe).
  float* red = reinterpret_cast<float*>(smem);
  const GemvWeight& G = a.w[wi];
  const int t_l = tid >> 4, cc = tid & 15;
  const int src = ((t_l >> 2) * 16 + cc) * 4 + (t_l & 3);
  float sums[NW][S][NT];
  constexpr bool kOnePass = NT * S * NW * W * 1024 <= 16384;
  if constexpr (kOnePass) {
    __syncthreads();  // every wave is past its LUT lookups
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int i = 0; i < S; ++i)
#pragma unroll
        for (int w = 0; w < NW; ++w)
          *reinterpret_cast<f32x4*>(red + ((((tt * S + i) * NW + w) * W + wave) * 64 + lane) * 4) = acc[w][i][tt];
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int i = 0; i < S; ++i)
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          float v = 0.0f;
          if (tid < 256) {
#pragma unroll
            for (int qq = 0; qq < W; ++qq) v += red[(((tt * S + i) * NW + w) * W + qq) * 256 + src];
          }
          sums[w][i][tt] = v;
        }
  } else {
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int i = 0; i < S; ++i) {
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; ++w)
          *reinterpret_cast<f32x4*>(red + ((w * W + wave) * 64 + lane) * 4) = acc[w][i][tt];
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          float v = 0.0f;
          if (tid < 256) {
#pragma unroll
            for (int qq = 0; qq < W; ++qq) v += red[(w * W + qq) * 256 + src];
          }
          sums[w][i][tt] = v;
        }
      }
  }
  const bool mine = tid < 256;
  if (P > 1) {
    // slab p's sums to the partials, then the last slab to arrive adds all
    // of them in slab order
    if (mine) {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        const int t = 16 * tt + t_l;
        if (t >= rows_arg) continue;
#pragma unroll
        for (int i = 0; i < S; ++i) {
          const size_t idx = ((size_t)p * rows_arg + t) * G.d_out + (s0 + i) * kStripeCols + cc;
#pragma unroll
          for (int w = 0; w < NW; ++w) store_coherent(&a.w[PAIR ? w : wi].partials[idx], sums[w][i][tt]);
        }
      }
    }
    wait_all_memory();
    int* is_last = reinterpret_cast<int*>(smem + kSkStageOffset);
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&G.counters[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *is_last = prev == (unsigned)(P - 1);
    }
    __syncthreads();
    if (!*is_last) return;
    if (mine) {
      // the partials of U slabs are all loaded before any of them is added
      // (the sum keeps slab order), so the hand-off costs one memory latency
      // per U slabs rather than one per slab
      constexpr int kVals = NT * S * NW;
      constexpr int U = kVals <= 8 ? 4 : kVals <= 16 ? 2 : 1;
      const size_t stride = (size_t)rows_arg * G.d_out;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int i = 0; i < S; ++i)
#pragma unroll
          for (int w = 0; w < NW; ++w) sums[w][i][tt] = 0.0f;
      for (int q0 = 0; q0 < P; q0 += U) {
        float pv[U][NT][S][NW];
#pragma unroll
        for (int dq = 0; dq < U; ++dq)
#pragma unroll
          for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < S; ++i)
#pragma unroll
              for (int w = 0; w < NW; ++w) {
                const int t = 16 * tt + t_l;
                const size_t idx = (size_t)t * G.d_out + (s0 + i) * kStripeCols + cc;
                pv[dq][tt][i][w] = (q0 + dq < P && t < rows_arg)
                                       ? load_coherent(a.w[PAIR ? w : wi].partials + idx + (q0 + dq) * stride)
                                       : 0.0f;
              }
#pragma unroll
        for (int dq = 0; dq < U; ++dq)
#pragma unroll
          for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < S; ++i)
#pragma unroll
              for (int w = 0; w < NW; ++w)
                if (q0 + dq < P) sums[w][i][tt] += pv[dq][tt][i][w];
      }
    }
    if (tid == 0) __hip_atomic_store(&G.counters[b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!mine) return;
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int t = 16 * tt + t_l;
    if (t >= rows_arg) continue;
    const float nrm = NORM ? inv_tok[tt * 16 + t_l] : 1.0f;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int gcol = (s0 + i) * kStripeCols + cc;
      float y = epilogue_value(G, sums[0][i][tt] * nrm, t, gcol);
      if constexpr (PAIR) y = silu_f32(y) * epilogue_value(a.w[1], sums[1][i][tt] * nrm, t, gcol);
      store_y(G, (size_t)t * G.d_out + gcol, y);
    }
  }
}

template <int NT, int W, int S, bool DQ, bool PAIR, bool XF32, bool NORM = false>
hipError_t sk_launch_t(const StripedArgs& a, int grid, int splits, hipStream_t stream) {
  constexpr int NW = PAIR ? 2 : 1;
  constexpr int D = (NT == 1 && S == 1) ? 4 : 2;
  constexpr int smem = kSkStageOffset + W * 512;
  static_assert(smem <= 65536, "skinny LDS");
  static_assert(W * NW * 1024 <= 16384, "the reduction reuses the LUT space below the norm's sums");
  static_assert(16384 + (NT * W * 16 + NT * 16) * 4 <= kLutBytes, "the norm's sums fit the LUT space");
  StripedArgs args = a;
  args.xcd_run = grid % 8 == 0 ? grid / 8 : 0;
  skinny_kernel<NT, W, D, S, DQ, PAIR, XF32, NORM><<<dim3(grid, splits), W * 64, smem, stream>>>(
      args.x, args.slot[0].packed, args.slot[0].scales, args.slot[0].scale_of_scales, args.d_in, args.rows_per_wave,
      args.rows_per_split, args.rows, args.xcd_run, args.nweights, splits, args.norm_w, args);
  return hipGetLastError();
}

// a folded norm (a.norm_w) takes the NORM kernels, built for double-quantized
// scales and whole-d_in grids (one slab)
template <int NT, int S, bool PAIR, bool XF32>
hipError_t sk_dispatch_w(const StripedArgs& a, int grid, int splits, int waves, bool dq, hipStream_t stream) {
  if (a.norm_w) {
    if (!dq || splits != 1) return hipErrorInvalidValue;
    if (waves == 4) return sk_launch_t<NT, 4, S, true, PAIR, XF32, true>(a, grid, splits, stream);
    if (waves == 8) return sk_launch_t<NT, 8, S, true, PAIR, XF32, true>(a, grid, splits, stream);
    return hipErrorInvalidValue;
  }
  if (waves == 4)
    return dq ? sk_launch_t<NT, 4, S, true, PAIR, XF32>(a, grid, splits, stream)
              : sk_launch_t<NT, 4, S, false, PAIR, XF32>(a, grid, splits, stream);
  if (waves == 8)
    return dq ? sk_launch_t<NT, 8, S, true, PAIR, XF32>(a, grid, splits, stream)
              : sk_launch_t<NT, 8, S, false, PAIR, XF32>(a, grid, splits, stream);
  return hipErrorInvalidValue;
}

template <int NT, bool PAIR, bool XF32>
hipError_t sk_dispatch_s(const StripedArgs& a, int grid, int splits, int waves, int group, bool dq,
                         hipStream_t stream) {
  if (group == 1) return sk_dispatch_w<NT, 1, PAIR, XF32>(a, grid, splits, waves, dq, stream);
  if (group == 2) return sk_dispatch_w<NT, 2, PAIR, XF32>(a, grid, splits, waves, dq, stream);
  if constexpr (!PAIR || NT == 1) {
    if (group == 4) return sk_dispatch_w<NT, 4, PAIR, XF32>(a, grid, splits, waves, dq, stream);
  }
  return hipErrorInvalidValue;
}

// token tiles of 16: 1, 2 or 4 (33..48 tokens run as four tiles)
int skinny_tiles(int rows) { return rows <= 16 ? 1 : rows <= 32 ? 2 : 4; }

// f32 activations take at most two token tiles (their 16 values per lane and
// tile fill the registers four tiles of bf16 take)
template <bool PAIR, bool XF32>
hipError_t sk_dispatch_rows(const StripedArgs& a, int grid, int splits, int waves, int group, bool dq,
                            hipStream_t stream) {
  switch (skinny_tiles(a.rows)) {
    case 1: return sk_dispatch_s<1, PAIR, XF32>(a, grid, splits, waves, group, dq, stream);
    case 2: return sk_dispatch_s<2, PAIR, XF32>(a, grid, splits, waves, group, dq, stream);
    case 4:
      if constexpr (!XF32) return sk_dispatch_s<4, PAIR, XF32>(a, grid, splits, waves, group, dq, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

StripedPlan plan_gemv_striped(int rows, int d_in, const int* d_out, int nweights, bool pair) {
  StripedPlan p{};
  int stripes = 0;
  for (int i = 0; i < (pair ? 1 : nweights); ++i) stripes += d_out[i] / kStripeCols;
  const int chunks = (d_in + 63) / 64;
  // About 4096 waves over the GPU (16 per CU): waves per workgroup = the
  // power of two at most 4096 / stripes, within [4, 16] (8 for the pair or
  // more than two rows, for registers) and no more than the 64-row chunks.
  // The pair's kernel takes ~140 VGPRs (three waves per SIMD): one 8-wave
  // workgroup per CU, so it keeps 4 waves (three workgroups per CU) once its
  // stripes pass 256, where 8 would run the grid in two rounds (Qwen2-0.5B
  // gate/up at one token: 9.9 -> 6.8 us).
  const int max_waves = pair ? (stripes > 256 ? 4 : 8) : rows > 2 ? 8 : 16;
  int waves = 4;
  while (waves < max_waves && (long)stripes * waves * 2 <= 4096 && waves * 2 <= chunks) waves *= 2;
  p.waves = waves;
  p.rows_per_wave = (chunks + waves - 1) / waves * 64;
  p.stripes = stripes;
  return p;
}

hipError_t launch_gemv_striped(const StripedPlan& p, const void* x, bool x_bf16, int rows, int d_in,
                               const GemvWeight* weights, int nweights, bool pair, hipStream_t stream,
                               const float* norm_w, float norm_eps) {
  StripedArgs a{};
  a.x = x;
  a.norm_w = norm_w;
  a.norm_eps = norm_eps;
  a.rows = rows;
  a.d_in = d_in;
  a.rows_per_wave = p.rows_per_wave;
  a.nweights = nweights;
  int s = 0;
  for (int i = 0; i < nweights; ++i) {
    a.w[i] = weights[i];
    a.stripe_begin[i] = pair ? 0 : s;
    if (!pair || i == 0) s += weights[i].d_out / kStripeCols;
  }
  for (int i = nweights; i <= kMaxGemvWeights; ++i) a.stripe_begin[i] = s;
  set_slots(a, weights, nweights);
  const bool dq = weights[0].scales.kind == kScalesDQ;
  if (pair) {
    if (rows == 1) return dispatch_w<1, true>(a, s, p.waves, x_bf16, dq, stream);
    if (rows == 2) return dispatch_w<2, true>(a, s, p.waves, x_bf16, dq, stream);
    return hipErrorInvalidValue;
  }
  switch (rows) {
    case 1: return dispatch_w<1, false>(a, s, p.waves, x_bf16, dq, stream);
    case 2: return dispatch_w<2, false>(a, s, p.waves, x_bf16, dq, stream);
    case 3: return dispatch_w<3, false>(a, s, p.waves, x_bf16, dq, stream);
    case 4: return dispatch_w<4, false>(a, s, p.waves, x_bf16, dq, stream);
    default: return hipErrorInvalidValue;
  }
}

bool skinny_supported(int rows, int d_in, const void* x, bool x_f32) {
  return rows >= 1 && rows <= (x_f32 ? kSkinnyMaxRowsF32 : kSkinnyMaxRows) && d_in > 0 && d_in % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
         (uint64_t)rows * (uint64_t)d_in * (x_f32 ? 4u : 2u) < (1ull << 31);
}

StripedPlan plan_skinny(int rows, int d_in, const int* d_out, int nweights, bool pair) {
  StripedPlan p{};
  int stripes = 0;
  for (int i = 0; i < (pair ? 1 : nweights); ++i) stripes += d_out[i] / kStripeCols;
  const int chunks = (d_in + 63) / 64;
  const int tiles = skinny_tiles(rows);
  // Stripes per wave (group): each activation load then feeds that many
  // stripes, which pays while the workgroups still cover the GPU (>= ~160);
  // the pair keeps its registers in bounds with two past one token tile.
  // With few stripes and a long d_in, d_in is split over workgroups (slabs
  // of >= 32 chunks) up to ~256 workgroups: the hand-off costs a few
  // microseconds of latency, which only a long d_in repays.
  const int g = (pair && tiles > 1) ? 2 : 4;
  int group = 1, splits = 1;
  if (tiles == 1 && chunks >= 64) {
    // one token tile over a long d_in: two stripes per wave and d_in slabs,
    // the pair in up to ~512 four-wave workgroups, a single weight in up to
    // ~256 eight-wave ones -- the same rows per wave, one LUT build per CU
    // and half the slabs to hand off (measured on the 7B-shaped MLP at 16
    // tokens: the gate/up pair 21.4 us against 24.1 us as 172 eight-wave
    // workgroups of four stripes; the block 34.7 us with down as 256
    // eight-wave workgroups over two slabs against 35.2-35.3 us as 512
    // four-wave ones over four)
    group = 2;
    const int waves = pair ? 4 : 8;
    while ((stripes / group) * splits < (pair ? 512 : 256) && chunks / (splits * 2) >= 32) splits *= 2;
    p.group = group;
    p.waves = waves;
    p.splits = splits;
    const int cps = (chunks + splits - 1) / splits;
    p.rows_per_wave = (cps + waves - 1) / waves * 64;
    p.rows_per_split = p.rows_per_wave * waves;
    p.stripes = stripes;
    return p;
  }
  if (stripes / g >= 160) {
    group = g;
  } else if (chunks >= 64) {
    // few stripes over a long d_in (the down projection of a decode batch):
    // fewer stripes per wave and slabs of >= 16 chunks, up to ~256
    // workgroups (Qwen2-0.5B down at 32 tokens: 28 -> 224 workgroups)
    group = stripes / g >= 64 ? g : stripes / 2 >= 64 ? 2 : 1;
    while ((stripes / group) * splits < 256 && chunks / (splits * 2) >= 16) splits *= 2;
  } else if (stripes / 2 >= 160) {
    group = 2;
  }
  const int waves = (tiles <= 2 && chunks / splits >= 16) ? 8 : 4;
  p.group = group;
  p.waves = waves;
  p.splits = splits;
  const int chunks_per_split = (chunks + splits - 1) / splits;
  p.rows_per_wave = (chunks_per_split + waves - 1) / waves * 64;
  p.rows_per_split = p.rows_per_wave * waves;
  p.stripes = stripes;
  return p;
}

hipError_t launch_skinny(const StripedPlan& p, const void* x, bool x_f32, int rows, int d_in,
                         const GemvWeight* weights, int nweights, bool pair, hipStream_t stream, const float* norm_w,
                         float norm_eps) {
  if (!skinny_supported(rows, d_in, x, x_f32) || nweights < 1 || nweights > kMaxGemvWeights || (pair && nweights != 2))
    return hipErrorInvalidValue;
  if ((p.group != 1 && p.group != 2 && p.group != 4) || p.splits < 1 || p.splits > 65535 ||
      (long)p.rows_per_split * p.splits < d_in || p.rows_per_split != p.rows_per_wave * p.waves)
    return hipErrorInvalidValue;
  StripedArgs a{};
  a.x = x;
  a.norm_w = norm_w;
  a.norm_eps = norm_eps;
  a.rows = rows;
  a.d_in = d_in;
  a.rows_per_wave = p.rows_per_wave;
  a.rows_per_split = p.rows_per_split;
  a.nweights = nweights;
  int s = 0;
  for (int i = 0; i < nweights; ++i) {
    a.w[i] = weights[i];
    if (p.splits > 1 && (!weights[i].partials || !weights[i].counters)) return hipErrorInvalidValue;
    a.stripe_begin[i] = pair ? 0 : s;
    if (!pair || i == 0) s += weights[i].d_out / kStripeCols;  // a multiple of 4: groups never straddle weights
  }
  for (int i = nweights; i <= kMaxGemvWeights; ++i) a.stripe_begin[i] = s;
  set_slots(a, weights, nweights);
  const bool dq = weights[0].scales.kind == kScalesDQ;
  const int grid = s / p.group;
  if (x_f32)
    return pair ? sk_dispatch_rows<true, true>(a, grid, p.splits, p.waves, p.group, dq, stream)
                : sk_dispatch_rows<false, true>(a, grid, p.splits, p.waves, p.group, dq, stream);
  return pair ? sk_dispatch_rows<true, false>(a, grid, p.splits, p.waves, p.group, dq, stream)
              : sk_dispatch_rows<false, false>(a, grid, p.splits, p.waves, p.group, dq, stream);
}

size_t skinny_partial_floats(const StripedPlan& p, int rows, int d_out) {
  return p.splits > 1 ? (size_t)p.splits * rows * d_out : 0;
}

}  // namespace unifur
