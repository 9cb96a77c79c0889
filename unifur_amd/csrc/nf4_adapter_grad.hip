// nf4_adapter_grad.hip -- the adapter gradients of the QLoRA backward on
// f32 matrix cores.
//
// For y = x W + s (x A) B (QLoraLinear::forward, src/qwennet.rs:325-345, with
// LoraAdapter::forward, src/quantize.rs:619-624) and dy = dL/dy, burn's
// autodiff under src/qwentrain.rs:421-470 gives the frozen base no gradient
// and the adapter
//     grad_b = (x A)^T (dy s)        [rank][N]
//     grad_a = x^T ((dy s) B^T)      [K][rank]
// Two launches compute them: the row products u = x A and t = dy B^T
// ([M][RB] f32, RB the rank rounded up to 16, 32 or 64, zero past the rank),
// then the column products grad_b = s u^T dy and grad_a = s x^T t.  Every
// product is a chain of v_mfma_f32_16x16x4f32 with bf16 inputs widened to
// f32 exactly, so the arithmetic is f32 throughout.  x and dy are each read
// twice; at rank 16 both launches are bound by those reads.
//
// MFMA operand layout (16 x 16 x 4): lane l = 16 g + i supplies A[i][g] and
// B[g][i] and receives D[4 g + e][i] in element e.  Each lane loads runs of
// eight consecutive values of its row and feeds them to consecutive MFMAs,
// so the reduction index lane group g covers at step s is
// k0 + 32 (s / 8) + 8 g + s % 8 (row products) and the output row MFMA q
// covers is v0 + 8 i + q (column products); the products are sums, so any
// fixed assignment is exact.
//
// Loads go through buffer resources bound to the workgroup's rows: a row
// past the slab or the tensor reads zero from the hardware bounds check, and
// a column or reduction index outside the slab is given an offset past every
// resource, so no load sits under a branch and a batch of them is issued
// before the MFMAs that consume it.
//
// Reductions are split over workgroups (slabs of K or N, or of M): the four
// waves of a workgroup add their sums through LDS in wave order, every slab
// writes its partial, and the last slab to arrive at a tile adds the
// partials in slab order -- the same bits whatever the arrival order.
#include "nf4_adapter_grad.hpp"

#include <algorithm>

#include "nf4_common.hpp"

namespace unifur {
namespace {

constexpr int kRowTile = 64;      // rows of x / dy per row-product workgroup
constexpr int kRowStep = 64;      // reduction values per wave step
constexpr int kColTile = 128;     // output rows (columns of x / dy) per column-product workgroup
constexpr int kColBatch = 8;      // 4-row steps whose loads a wave issues together
constexpr int kRowGrid = 512;     // workgroups the row launch aims for (two products)
constexpr int kColGrid = 512;     // and the column launch
constexpr int kMaxSlabs = 32;
constexpr uint32_t kOob = 0x80000000u;  // an offset past every resource (all stay below 2^31 bytes)
constexpr int kRsrcWord3 = 0x00020000;  // raw-buffer descriptor word 3

int rank_bucket(int rank) { return rank <= 16 ? 16 : rank <= 32 ? 32 : 64; }
int cdiv(int a, int b) { return (a + b - 1) / b; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

// Eight consecutive values at byte offset off, as loaded: bf16 pairs in four
// dwords, or f32 in eight.
template <bool BF16>
struct Run8 {
  u32x4 v[BF16 ? 1 : 2];
};

template <bool BF16>
__device__ __forceinline__ Run8<BF16> load_run8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  Run8<BF16> o;
  o.v[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  if constexpr (!BF16) o.v[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16u, 0, 0));
  return o;
}

// element e of a run, widened to f32 (bf16 exactly)
template <bool BF16>
__device__ __forceinline__ float run_at(const Run8<BF16>& r, int e) {
  if constexpr (BF16) {
    const uint32_t w = r.v[0][e >> 1];
    return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return __uint_as_float(r.v[e >> 2][e & 3]);
  }
}

// Eight f32 values as three bf16x8 terms whose sum is exact: hi = bf16(w),
// mid = bf16(w - hi), lo = w - hi - mid (each difference is exact in f32 and
// the last fits bf16's eight significand bits).
__device__ __forceinline__ void split3_bf16(const float* w, u32x4 (&parts)[3]) {
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = w[e];
#pragma unroll
  for (int t = 0; t < 3; ++t) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t pk = pack_bf16x2(r[2 * e], r[2 * e + 1]);
      parts[t][e] = pk;
      r[2 * e] -= __uint_as_float(pk << 16);
      r[2 * e + 1] -= __uint_as_float(pk & 0xffff0000u);
    }
  }
}

// The last slab's sums over the partials of all slabs, in slab order:
// sums[i] = partials[0][off[i]] + partials[1][off[i]] + ... for this
// thread's N values.  The coherent loads of eight slabs are issued before
// any of them is added, so the hand-off costs a few memory latencies rather
// than one per slab and value.
template <int N>
__device__ __forceinline__ void sum_slabs(const float* partials, size_t slab_stride, int slabs, const size_t (&off)[N],
                                          const bool (&live)[N], float (&sums)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) sums[i] = 0.0f;
  for (int q0 = 0; q0 < slabs; q0 += 8) {
    float t[8][N];
#pragma unroll
    for (int dq = 0; dq < 8; ++dq)
#pragma unroll
      for (int i = 0; i < N; ++i)
        t[dq][i] = (q0 + dq < slabs && live[i]) ? load_coherent(partials + (size_t)(q0 + dq) * slab_stride + off[i])
                                                 : 0.0f;
#pragma unroll
    for (int dq = 0; dq < 8; ++dq)
#pragma unroll
      for (int i = 0; i < N; ++i)
        if (q0 + dq < slabs) sums[i] += t[dq][i];
  }
}

// ------------------------------------------------------------ row products --

// out_p[m][j] = sum_k src_p[m][k] w_p(k, j) for p = blockIdx.z + first:
// p = 0: x [M][K] with A [K][rank] (w(k, j) = A[k][j]) -> u;
// p = 1: dy [M][N] with B [rank][N] (w(k, j) = B[j][k]) -> t.
struct RowArgs {
  const void* src[2];
  const float* w[2];
  int kdim[2], slabs[2], kslab[2];
  float* out[2];       // [M][RB]
  float* partials[2];  // [slabs][M][RB]
  unsigned* counters[2];
  int M, rank, first;
};

constexpr int kRowRed = 17;  // LDS row pitch of the wave sums (floats)

template <bool BF16, int RB, bool W_KMAJOR>
__device__ __forceinline__ void row_body(const RowArgs& a, int p, float* red, int* flag) {
  constexpr int JB = RB / 16;
  constexpr uint32_t esz = BF16 ? 2 : 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, g = lane >> 4;
  const int M = a.M, kd = a.kdim[p], slabs = a.slabs[p], slab = blockIdx.y, rank = a.rank;
  const int m0 = blockIdx.x * kRowTile;
  const int kb = slab * a.kslab[p], ke = min(kd, kb + a.kslab[p]);
  const int rows = min(kRowTile, M - m0);
  const __amdgpu_buffer_rsrc_t xr =
      make_rsrc(static_cast<const char*>(a.src[p]) + (size_t)m0 * kd * esz, (uint32_t)rows * (uint32_t)kd * esz);
  // A: the slab's rows [kb, ke) of [K][rank]; B: all of [rank][N]
  const __amdgpu_buffer_rsrc_t wr =
      W_KMAJOR ? make_rsrc(a.w[p] + (size_t)kb * rank, (uint32_t)(ke - kb) * (uint32_t)rank * 4u)
               : make_rsrc(a.w[p], (uint32_t)rank * (uint32_t)kd * 4u);
  f32x4 acc[4][JB];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) acc[rb][jb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // U steps per iteration: the loads of all of them are issued before the
  // first MFMA (one step at rank 64, where the operands fill the registers)
  constexpr int U = JB == 1 ? 2 : 1;
  for (int k1 = kb + wave * kRowStep; k1 < ke; k1 += U * 4 * kRowStep) {
    Run8<BF16> xv[U][4][2];
    float wv[U][JB][16];
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      const int k0 = k1 + uu * 4 * kRowStep;
      // A operand: row 16 rb + i16, runs at k0 + 32 h + 8 g (ke is a multiple
      // of 8, so a run is wholly inside or outside the slab)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = k0 + 32 * h + 8 * g;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
          xv[uu][rb][h] =
              load_run8<BF16>(xr, k < ke ? ((uint32_t)(16 * rb + i16) * (uint32_t)kd + (uint32_t)k) * esz : kOob);
      }
      // B operand: w(k, 16 jb + i16) at the same k
      if constexpr (W_KMAJOR) {
#pragma unroll
        for (int jb = 0; jb < JB; ++jb) {
          const int j = 16 * jb + i16;
#pragma unroll
          for (int s = 0; s < 16; ++s) {
            const int k = k0 + 32 * (s >> 3) + 8 * g + (s & 7);
            wv[uu][jb][s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                wr, j < rank && k < ke ? ((uint32_t)(k - kb) * (uint32_t)rank + (uint32_t)j) * 4u : kOob, 0, 0));
          }
        }
      } else {
#pragma unroll
        for (int jb = 0; jb < JB; ++jb) {
          const int j = 16 * jb + i16;  // rows j >= rank fall outside wr
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int k = k0 + 32 * h + 8 * g;
            const Run8<false> r =
                load_run8<false>(wr, k < ke ? ((uint32_t)j * (uint32_t)kd + (uint32_t)k) * 4u : kOob);
#pragma unroll
            for (int e = 0; e < 8; ++e) wv[uu][jb][8 * h + e] = run_at<false>(r, e);
          }
        }
      }
    }
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      if (k1 + uu * 4 * kRowStep >= ke) break;  // uniform: past the slab the loads read zero
      if constexpr (BF16) {
        // a run of eight bf16 values is the A operand of v_mfma_f32_16x16x32_bf16
        // as loaded; w splits exactly into three bf16 terms (hi + mid + lo
        // carry its 24 significand bits), so three bf16 products give the f32
        // product
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int jb = 0; jb < JB; ++jb) {
            u32x4 parts[3];
            split3_bf16(&wv[uu][jb][8 * h], parts);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
              for (int t = 2; t >= 0; --t)
                acc[rb][jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, xv[uu][rb][h].v[0]), __builtin_bit_cast(bf16x8_t, parts[t]),
                    acc[rb][jb], 0, 0, 0);
          }
      } else {
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
          for (int rb = 0; rb < 4; ++rb) {
            const float xs = run_at<BF16>(xv[uu][rb][s >> 3], s & 7);
#pragma unroll
            for (int jb = 0; jb < JB; ++jb)
              acc[rb][jb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs, wv[uu][jb][s], acc[rb][jb], 0, 0, 0);
          }
      }
    }
  }

  // the four waves' sums in wave order; one slab's partial or the result
  float* out = a.out[p];
  float* part = a.partials[p] + (size_t)slab * M * RB;
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[(wave * kRowTile + 16 * rb + 4 * g + e) * kRowRed + i16] = acc[rb][jb][e];
    __syncthreads();
    for (int i = tid; i < kRowTile * 16; i += 256) {
      const int r = i >> 4, c = i & 15;
      float v = red[r * kRowRed + c];
#pragma unroll
      for (int q = 1; q < 4; ++q) v += red[(q * kRowTile + r) * kRowRed + c];
      if (r < rows) {
        const size_t o = (size_t)(m0 + r) * RB + 16 * jb + c;
        if (slabs == 1) out[o] = v;
        else store_coherent(&part[o], v);
      }
    }
    __syncthreads();
  }
  if (slabs == 1) return;
  wait_all_memory();
  __syncthreads();
  unsigned* counter = &a.counters[p][blockIdx.x];
  if (tid == 0) *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        (unsigned)(slabs - 1);
  __syncthreads();
  if (!*flag) return;
  constexpr int VPT = kRowTile * RB / 256;  // values per thread
  size_t off[VPT];
  bool live[VPT];
  float sums[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = tid + 256 * i;
    off[i] = (size_t)m0 * RB + idx;
    live[i] = idx < rows * RB;
  }
  sum_slabs<VPT>(a.partials[p], (size_t)M * RB, slabs, off, live, sums);
#pragma unroll
  for (int i = 0; i < VPT; ++i)
    if (live[i]) out[off[i]] = sums[i];
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool BF_X, bool BF_DY, int RB>
__global__ __launch_bounds__(256) void row_products_kernel(RowArgs a) {
  __shared__ float red[4 * kRowTile * kRowRed];
  __shared__ int flag;
  const int p = (int)blockIdx.z + a.first;
  if ((int)blockIdx.y >= a.slabs[p]) return;  // the other product has more slabs
  if (p == 0) row_body<BF_X, RB, true>(a, 0, red, &flag);
  else row_body<BF_DY, RB, false>(a, 1, red, &flag);
}

// --------------------------------------------------------- column products --

// out_p(v, j) = scale sum_m wide_p[m][v] nar_p[m][j] for v < width_p,
// j < rank, p = blockIdx.z + first: p = 0: (dy, u) -> grad_b [rank][N];
// p = 1: (x, t) -> grad_a [K][rank].
struct ColArgs {
  const void* wide[2];
  const float* nar[2];  // [M][RB]
  int width[2];
  float* out[2];
  float* partials[2];  // [slabs][RB][width] (p = 0) or [slabs][width][RB] (p = 1)
  unsigned* counters[2];
  int slabs, mslab, M, rank, first;
  float scale;
};

constexpr int kColRed = 17;

template <bool BF16, int RB, bool NAR_MAJOR>
__device__ __forceinline__ void col_body(const ColArgs& a, int p, float* red, int* flag) {
  constexpr int JB = RB / 16;
  constexpr uint32_t esz = BF16 ? 2 : 4;
  const int W = a.width[p];
  const int v0 = blockIdx.x * kColTile;
  if (v0 >= W) return;  // the other product is wider; uniform over the workgroup
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, g = lane >> 4;
  const int M = a.M, slabs = a.slabs, slab = blockIdx.y, rank = a.rank;
  const int mb = slab * a.mslab;
  const int rows = max(0, min(a.mslab, M - mb));
  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(static_cast<const char*>(a.wide[p]) + (size_t)mb * W * esz, (uint32_t)rows * (uint32_t)W * esz);
  const __amdgpu_buffer_rsrc_t nr = make_rsrc(a.nar[p] + (size_t)mb * RB, (uint32_t)rows * RB * 4u);
  const int vl = v0 + 8 * i16;  // this lane's eight columns (W % 8 == 0)
  const bool vok = vl < W;
  f32x4 acc[8][JB];
#pragma unroll
  for (int q = 0; q < 8; ++q)
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) acc[q][jb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // wave w takes the 4-row steps w, w + 4, ...: rows 4 w + 16 i + g
  for (int m = 4 * wave; m < rows; m += 16 * kColBatch) {
    Run8<BF16> wv[kColBatch];
    float nv[kColBatch][JB];
#pragma unroll
    for (int u = 0; u < kColBatch; ++u) {
      const uint32_t r = (uint32_t)(m + 16 * u + g);  // rows past the slab fall outside wr and nr
      wv[u] = load_run8<BF16>(wr, vok ? (r * (uint32_t)W + (uint32_t)vl) * esz : kOob);
#pragma unroll
      for (int jb = 0; jb < JB; ++jb)
        nv[u][jb] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(nr, (r * RB + 16 * jb + i16) * 4u, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < kColBatch; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float ws = run_at<BF16>(wv[u], q);
#pragma unroll
        for (int jb = 0; jb < JB; ++jb)
          acc[q][jb] = __builtin_amdgcn_mfma_f32_16x16x4f32(ws, nv[u][jb], acc[q][jb], 0, 0, 0);
      }
  }

  float* out = a.out[p];
  float* part = a.partials[p] + (size_t)slab * W * RB;
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) {
    // element e of MFMA q in lane 16 g + i16: v = v0 + 8 (4 g + e) + q, j = 16 jb + i16
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[(wave * kColTile + 8 * (4 * g + e) + q) * kColRed + i16] = acc[q][jb][e];
    __syncthreads();
    for (int i = tid; i < kColTile * 16; i += 256) {
      // consecutive threads take consecutive v for the [rank][width] layout
      const int r = NAR_MAJOR ? i % kColTile : i >> 4, c = NAR_MAJOR ? i / kColTile : i & 15;
      float v = red[r * kColRed + c];
#pragma unroll
      for (int q = 1; q < 4; ++q) v += red[(q * kColTile + r) * kColRed + c];
      const int vv = v0 + r, j = 16 * jb + c;
      if (vv < W) {
        // partials laid out like the output ([j][v] or [v][j]), so that
        // consecutive threads store and load consecutive words
        if (slabs > 1) store_coherent(&part[NAR_MAJOR ? (size_t)j * W + vv : (size_t)vv * RB + j], v);
        else if (j < rank) out[NAR_MAJOR ? (size_t)j * W + vv : (size_t)vv * rank + j] = v * a.scale;
      }
    }
    __syncthreads();
  }
  if (slabs == 1) return;
  wait_all_memory();
  __syncthreads();
  unsigned* counter = &a.counters[p][blockIdx.x];
  if (tid == 0) *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        (unsigned)(slabs - 1);
  __syncthreads();
  if (!*flag) return;
  // eight values per thread at a time; consecutive threads take consecutive
  // v for the [rank][width] layout
  constexpr int VPT = 8;
  for (int i0 = 0; i0 < kColTile * RB; i0 += 256 * VPT) {
    size_t off[VPT];
    bool live[VPT];
    float sums[VPT];
    int vvs[VPT], js[VPT];
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
      const int i = i0 + tid + 256 * e;
      const int r = NAR_MAJOR ? i % kColTile : i / RB, j = NAR_MAJOR ? i / kColTile : i % RB;
      vvs[e] = v0 + r;
      js[e] = j;
      live[e] = i < kColTile * RB && v0 + r < W && j < rank;
      off[e] = NAR_MAJOR ? (size_t)j * W + v0 + r : (size_t)(v0 + r) * RB + j;
    }
    sum_slabs<VPT>(a.partials[p], (size_t)W * RB, slabs, off, live, sums);
#pragma unroll
    for (int e = 0; e < VPT; ++e)
      if (live[e]) out[NAR_MAJOR ? (size_t)js[e] * W + vvs[e] : (size_t)vvs[e] * rank + js[e]] = sums[e] * a.scale;
  }
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool BF_X, bool BF_DY, int RB>
__global__ __launch_bounds__(256) void col_products_kernel(ColArgs a) {
  __shared__ float red[4 * kColTile * kColRed];
  __shared__ int flag;
  if ((int)blockIdx.z + a.first == 0) col_body<BF_DY, RB, true>(a, 0, red, &flag);
  else col_body<BF_X, RB, false>(a, 1, red, &flag);
}

// ------------------------------------------------------------------ plan --

// Slab counts depend only on the shapes (both products assumed), so the
// workspace query and the launch agree.
struct Plan {
  int rb, row_tiles, row_slabs[2], row_kslab[2], col_tiles[2], col_slabs, col_mslab;
  size_t u, t, row_part[2], col_part[2], partials, total;  // scratch offsets / bytes
};

size_t align256(size_t b) { return (b + 255) & ~size_t{255}; }

Plan make_plan(int M, int K, int N, int rank) {
  Plan P{};
  P.rb = rank_bucket(rank);
  P.row_tiles = cdiv(M, kRowTile);
  const int kd[2] = {K, N}, wd[2] = {N, K};
  size_t row_part = 0, col_part = 0;
  for (int p = 0; p < 2; ++p) {
    int slabs = P.row_tiles > 0 ? cdiv(kRowGrid / 2, P.row_tiles) : 1;
    slabs = std::max(1, std::min(std::min(slabs, kMaxSlabs), cdiv(kd[p], 4 * kRowStep)));
    const int kslab = std::max(1, cdiv(cdiv(kd[p], slabs), 4 * kRowStep)) * 4 * kRowStep;
    P.row_kslab[p] = kslab;
    P.row_slabs[p] = std::max(1, cdiv(kd[p], kslab));
    P.row_part[p] = P.row_slabs[p] > 1 ? align256((size_t)P.row_slabs[p] * M * P.rb * sizeof(float)) : 0;
    row_part += P.row_part[p];
    P.col_tiles[p] = cdiv(wd[p], kColTile);
  }
  int slabs = cdiv(kColGrid, P.col_tiles[0] + P.col_tiles[1]);
  slabs = std::max(1, std::min(std::min(slabs, kMaxSlabs), cdiv(M, 64)));
  P.col_mslab = M > 0 ? cdiv(cdiv(M, slabs), 16) * 16 : 16;
  P.col_slabs = M > 0 ? cdiv(M, P.col_mslab) : 1;
  for (int p = 0; p < 2; ++p) {
    P.col_part[p] = P.col_slabs > 1 ? align256((size_t)P.col_slabs * wd[p] * P.rb * sizeof(float)) : 0;
    col_part += P.col_part[p];
  }
  P.u = 0;
  P.t = align256((size_t)M * P.rb * sizeof(float));
  P.partials = P.t + align256((size_t)M * P.rb * sizeof(float));
  P.total = P.partials + std::max(row_part, col_part);
  return P;
}

template <int RB>
hipError_t launch_rows(const RowArgs& a, bool bx, bool bdy, dim3 grid, hipStream_t s) {
  if (bx) {
    if (bdy) row_products_kernel<true, true, RB><<<grid, 256, 0, s>>>(a);
    else row_products_kernel<true, false, RB><<<grid, 256, 0, s>>>(a);
  } else {
    if (bdy) row_products_kernel<false, true, RB><<<grid, 256, 0, s>>>(a);
    else row_products_kernel<false, false, RB><<<grid, 256, 0, s>>>(a);
  }
  return hipGetLastError();
}

template <int RB>
hipError_t launch_cols(const ColArgs& a, bool bx, bool bdy, dim3 grid, hipStream_t s) {
  if (bx) {
    if (bdy) col_products_kernel<true, true, RB><<<grid, 256, 0, s>>>(a);
    else col_products_kernel<true, false, RB><<<grid, 256, 0, s>>>(a);
  } else {
    if (bdy) col_products_kernel<false, true, RB><<<grid, 256, 0, s>>>(a);
    else col_products_kernel<false, false, RB><<<grid, 256, 0, s>>>(a);
  }
  return hipGetLastError();
}

}  // namespace

bool adapter_grads_supported(const void* x, const void* dy, const float* b, int M, int K, int N, int rank) {
  const auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (rank < 1 || rank > 64 || M < 0 || K <= 0 || N <= 0 || K % 8 || N % 8 || !al(x) || !al(dy) || !al(b))
    return false;
  // every buffer resource (and every offset a load forms past one) stays
  // below 2^31 bytes: a row tile of x or dy, B, a column slab plus a batch
  const Plan P = make_plan(M, K, N, rank);
  const uint64_t widest = (uint64_t)std::max(K, N) * 4u;
  return widest * (kRowTile + 64) < (1ull << 31) &&
         widest * (uint64_t)(P.col_mslab + 16 * kColBatch + 16) < (1ull << 31);
}

size_t adapter_grads_scratch_bytes(int M, int K, int N, int rank) { return make_plan(M, K, N, rank).total; }

int adapter_row_product_ld(int rank) { return rank_bucket(rank); }

bool adapter_row_product_supported(const void* src, const float* w, int M, int kdim, int rank) {
  return adapter_grads_supported(src, src, w, M, kdim, kdim, rank);
}

size_t adapter_row_product_scratch_bytes(int M, int kdim, int rank) {
  const Plan P = make_plan(M, kdim, kdim, rank);
  return align256((size_t)M * P.rb * sizeof(float)) + P.row_part[0];
}

hipError_t launch_adapter_row_product(int p, const void* src, bool src_bf16, const float* w, int M, int kdim,
                                      int rank, void* scratch, unsigned* counters, int max_counters,
                                      hipStream_t stream) {
  if ((p != 0 && p != 1) || !adapter_row_product_supported(src, w, M, kdim, rank)) return hipErrorInvalidValue;
  if (M == 0) return hipSuccess;
  const Plan P = make_plan(M, kdim, kdim, rank);  // both products over kdim: the same slabs
  char* base = static_cast<char*>(scratch);
  RowArgs ra{};
  for (int q = 0; q < 2; ++q) {
    ra.src[q] = src;
    ra.w[q] = w;
    ra.kdim[q] = kdim;
    ra.out[q] = reinterpret_cast<float*>(base);
    ra.partials[q] = reinterpret_cast<float*>(base + align256((size_t)M * P.rb * sizeof(float)));
    ra.counters[q] = counters;
    ra.slabs[q] = P.row_slabs[q];
    ra.kslab[q] = P.row_kslab[q];
  }
  ra.M = M, ra.rank = rank, ra.first = p;
  if (P.row_slabs[p] > 1 && P.row_tiles > max_counters) return hipErrorInvalidValue;
  const dim3 grid((unsigned)P.row_tiles, (unsigned)P.row_slabs[p], 1u);
  return P.rb == 16   ? launch_rows<16>(ra, src_bf16, src_bf16, grid, stream)
         : P.rb == 32 ? launch_rows<32>(ra, src_bf16, src_bf16, grid, stream)
                      : launch_rows<64>(ra, src_bf16, src_bf16, grid, stream);
}

hipError_t launch_adapter_grads(const void* x, bool x_bf16, const void* dy, bool dy_bf16, const float* a,
                                const float* b, int M, int K, int N, int rank, float scaling, float* grad_a,
                                float* grad_b, void* scratch, unsigned* counters, int max_counters,
                                hipStream_t stream) {
  if (!grad_a && !grad_b) return hipSuccess;
  if (!adapter_grads_supported(x, dy, b, M, K, N, rank) || (M > 0 && (!x || !dy)) || !a || !b)
    return hipErrorInvalidValue;
  const Plan P = make_plan(M, K, N, rank);
  char* base = static_cast<char*>(scratch);
  float* u = reinterpret_cast<float*>(base + P.u);
  float* t = reinterpret_cast<float*>(base + P.t);
  float* part = reinterpret_cast<float*>(base + P.partials);

  // product 0: (x, A) -> u, then (dy, u) -> grad_b; product 1: (dy, B^T) ->
  // t, then (x, t) -> grad_a.  The launches cover products first .. last.
  const int first = grad_b ? 0 : 1, last = grad_a ? 1 : 0, nprod = last - first + 1;
  RowArgs ra{};
  ra.src[0] = x, ra.src[1] = dy;
  ra.w[0] = a, ra.w[1] = b;
  ra.kdim[0] = K, ra.kdim[1] = N;
  ra.out[0] = u, ra.out[1] = t;
  ra.partials[0] = part, ra.partials[1] = part + P.row_part[0] / sizeof(float);
  ra.M = M, ra.rank = rank, ra.first = first;
  ColArgs ca{};
  ca.wide[0] = dy, ca.wide[1] = x;
  ca.nar[0] = u, ca.nar[1] = t;
  ca.width[0] = N, ca.width[1] = K;
  ca.out[0] = grad_b, ca.out[1] = grad_a;
  ca.partials[0] = part, ca.partials[1] = part + P.col_part[0] / sizeof(float);
  ca.slabs = P.col_slabs, ca.mslab = P.col_mslab, ca.M = M, ca.rank = rank, ca.first = first;
  ca.scale = scaling;
  int row_slabs = 1, col_tiles = 1, row_counters = 0, col_counters = 0;
  for (int p = first; p <= last; ++p) {
    ra.slabs[p] = P.row_slabs[p], ra.kslab[p] = P.row_kslab[p];
    ra.counters[p] = counters + row_counters;
    row_counters += P.row_tiles;
    row_slabs = std::max(row_slabs, P.row_slabs[p]);
    ca.counters[p] = counters + col_counters;
    col_counters += P.col_tiles[p];
    col_tiles = std::max(col_tiles, P.col_tiles[p]);
  }
  // counters are only touched by split reductions, which the plan keeps to
  // fewer than a launch's target of workgroups
  if ((row_slabs > 1 && row_counters > max_counters) || (P.col_slabs > 1 && col_counters > max_counters))
    return hipErrorInvalidValue;

  if (M > 0) {
    const dim3 grid((unsigned)P.row_tiles, (unsigned)row_slabs, (unsigned)nprod);
    const hipError_t e = P.rb == 16   ? launch_rows<16>(ra, x_bf16, dy_bf16, grid, stream)
                         : P.rb == 32 ? launch_rows<32>(ra, x_bf16, dy_bf16, grid, stream)
                                      : launch_rows<64>(ra, x_bf16, dy_bf16, grid, stream);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((unsigned)col_tiles, (unsigned)P.col_slabs, (unsigned)nprod);
  return P.rb == 16   ? launch_cols<16>(ca, x_bf16, dy_bf16, grid, stream)
         : P.rb == 32 ? launch_cols<32>(ca, x_bf16, dy_bf16, grid, stream)
                      : launch_cols<64>(ca, x_bf16, dy_bf16, grid, stream);
}

}  // namespace unifur
