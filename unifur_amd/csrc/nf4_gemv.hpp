// nf4_gemv.hpp -- internal interface of the decode GEMV (few input rows).
#pragma once

#include "nf4_codec.hpp"

namespace unifur {

constexpr int kMaxGemvWeights = 3;

// One NF4 weight [d_in, d_out] of a (possibly batched) GEMV launch.
struct GemvWeight {
  const uint8_t* packed;  // ceil(d_in * d_out / 2) bytes
  ScalesArg scales;
  int d_out;
  void* y;  // [rows, d_out] f32 or bf16
  int y_bf16;
  const float* bias;     // [d_out] or null
  const float* lora_xa;  // [rows, lora_rank] = x A, or null
  const float* lora_b;   // [lora_rank, d_out]
  int lora_rank;
  float lora_scaling;
  unsigned* counters;  // workspace: one zeroed u32 per 256-column tile
  float* partials;     // workspace: splits * rows * d_out floats (split-K)
  const void* residual;  // striped GEMV / skinny: [rows, d_out] in y's dtype added last, or null
};

struct GemvPlan {
  bool pair;  // gate/up SwiGLU pair: weights[0], weights[1] share x and d_out
  int rows_per_thread;
  int rows_per_wg;
  int splits;
  int tiles;
  int counter_count[kMaxGemvWeights];
  size_t partial_count[kMaxGemvWeights];
};

constexpr int kGemvMaxRows = 4;      // activation rows handled by the GEMV path
constexpr int kGemvPairMaxRows = 2;  // ... and by its SwiGLU gate/up pair mode

// Plan a launch over nweights weights sharing x [rows, d_in]; with pair, the
// two weights are gate and up of a SwiGLU block and weights[0].y receives
// silu(gate x) * (up x).
GemvPlan plan_gemv(int rows, int d_in, const int* d_out, int nweights, bool pair);

hipError_t launch_gemv(const GemvPlan& p, const void* x, bool x_bf16, int rows, int d_in, const GemvWeight* weights,
                       int nweights, hipStream_t stream);

// ---- the same GEMV over weights in the striped layout (nf4_layout.hpp) ----
// No workspace: each workgroup reduces its 16-column stripe over all of d_in.
// d_out of every weight a multiple of 64; x [rows, d_in], rows in 1..4 (1..2
// for the SwiGLU pair); the GemvWeight fields counters and partials are unused.

struct StripedPlan {
  int waves;          // waves per workgroup: 4, 8 or 16
  int rows_per_wave;  // a multiple of 64
  int stripes;        // stripes of the launch (workgroups = stripes / group)
  int group;          // skinny kernel: stripes per wave (1, 2 or 4); the GEMV takes 1
  int splits;         // skinny kernel: d_in slabs over workgroups (1 for the GEMV)
  int rows_per_split; // skinny kernel: waves * rows_per_wave
};

// What the first loads of a striped launch need of weight slot i.  With the
// shape fields and stripe_begin these lie in the first two 64-byte lines of
// the arguments, so that the prologue's argument loads miss the scalar cache
// at most once; the full GemvWeight records, which the epilogue reads, follow.
struct StripedSlot {
  const uint8_t* packed;
  const void* scales;  // u8 DQ codes or f32 absmax, as the weight's scale kind
  const float* scale_of_scales;
};

struct StripedArgs {
  const void* x;  // [rows, d_in] f32 or bf16
  int rows;
  int d_in;
  int rows_per_wave;
  int rows_per_split;  // skinny kernel: d_in rows per workgroup along gridDim.y
  int nweights;
  // XCD-aware order: gridDim.x / 8 when that divides evenly, else 0 (set by
  // the launcher, so that the kernels need not read the grid size first)
  int xcd_run;
  StripedSlot slot[kMaxGemvWeights];
  int stripe_begin[kMaxGemvWeights + 1];  // prefix sums of stripes per weight
  GemvWeight w[kMaxGemvWeights];
  // QwenRmsNorm folded into the launch, x -> x * rsqrt(mean(x^2) +
  // norm_eps) * (norm_w + 1) per row
  const float* norm_w;  // [d_in] or null
  float norm_eps;
};

StripedPlan plan_gemv_striped(int rows, int d_in, const int* d_out, int nweights, bool pair);

// norm_w != null folds QwenRmsNorm (weight norm_w, epsilon norm_eps) over x
// into the launch: each workgroup sums x^2 over all of d_in beside the
// products and scales its results by the row's 1 / sqrt(mean + eps).
hipError_t launch_gemv_striped(const StripedPlan& p, const void* x, bool x_bf16, int rows, int d_in,
                               const GemvWeight* weights, int nweights, bool pair, hipStream_t stream,
                               const float* norm_w = nullptr, float norm_eps = 0.0f);

// ---- 5..64 bf16 rows (5..32 f32 rows) over striped weights, on MFMA ----
// Same decomposition (a workgroup per stripe over all of d_in, waves split
// d_in) with the products on MFMA: for bf16 x v_mfma_f32_16x16x32_bf16 with
// the weight operand bf16(level * scale) (the rounding of the MFMA GEMM
// path); for f32 x v_mfma_f32_16x16x4_f32 with the weight operand the exact
// f32 level * scale (the reference's dequantized value).  x is used as it
// is.  Needs d_in % 8 == 0, x 16-byte aligned, rows * d_in * sizeof(x) under
// 2^31; the SwiGLU pair mode stores silu(gate x) * (up x).  With
// plan.splits > 1 the workgroups of a stripe group split d_in and hand their
// partial sums over through the GemvWeight fields partials (splits * rows *
// d_out floats per weight) and counters (one zeroed u32 per stripe group,
// left zeroed): the last to arrive adds them in slab order.
constexpr int kSkinnyMaxRows = 64;
constexpr int kSkinnyMaxRowsF32 = 32;

bool skinny_supported(int rows, int d_in, const void* x, bool x_f32 = false);

StripedPlan plan_skinny(int rows, int d_in, const int* d_out, int nweights, bool pair);

// norm_w != null folds QwenRmsNorm (weight norm_w, epsilon norm_eps) over x
// into the launch, as the GEMV does: needs double-quantized scales and a
// plan without d_in slabs (plan.splits == 1).
hipError_t launch_skinny(const StripedPlan& p, const void* x, bool x_f32, int rows, int d_in,
                         const GemvWeight* weights, int nweights, bool pair, hipStream_t stream,
                         const float* norm_w = nullptr, float norm_eps = 0.0f);

// floats of GemvWeight::partials one weight of a skinny launch needs (0 without splits)
size_t skinny_partial_floats(const StripedPlan& p, int rows, int d_out);

}  // namespace unifur
