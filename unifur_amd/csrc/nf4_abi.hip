// nf4_abi.hip -- the extern "C" boundary (include/unifur_nf4.h).
//
// Argument validation, path selection, workspace carving and error
// reporting; every computation is a launch of a kernel in this library.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "../../include/unifur_nf4.h"
#include "nf4_adapter_grad.hpp"
#include "nf4_codec.hpp"
#include "nf4_embedding.hpp"
#include "nf4_expand.hpp"
#include "nf4_gemm.hpp"
#include "nf4_gemm_f32.hpp"
#include "nf4_generic.hpp"
#include "nf4_gemv.hpp"
#include "nf4_layout.hpp"

namespace unifur {
namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int fail_hip(hipError_t e, const char* what) {
  return fail(UNIFUR_NF4_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define UNIFUR_ARG(cond, msg) \
  do {                        \
    if (!(cond)) return fail(UNIFUR_NF4_ERR_INVALID, msg); \
  } while (0)

#define UNIFUR_HIP(expr)                          \
  do {                                            \
    hipError_t e_ = (expr);                       \
    if (e_ != hipSuccess) return fail_hip(e_, #expr); \
  } while (0)

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
uint64_t ceil_div_u64(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

bool u32_aligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

bool valid_dtype(int d) { return d == UNIFUR_NF4_F32 || d == UNIFUR_NF4_BF16; }

// Element types a checkpoint tensor may arrive in (src/import.rs:255-272):
// F32, BF16 and F16, each decoded to f32 exactly.  Only the checkpoint
// entry points take F16; activations are f32 or bf16.
bool valid_src_dtype(int d) { return d == UNIFUR_NF4_F32 || d == UNIFUR_NF4_BF16 || d == UNIFUR_NF4_F16; }
int src_kind_of(int d) { return d == UNIFUR_NF4_BF16 ? kSrcBf16 : d == UNIFUR_NF4_F16 ? kSrcF16 : kSrcF32; }

ScalesArg to_scales(const unifur_nf4_scales& s) {
  return ScalesArg{s.kind, s.absmax, s.dq_codes, s.scale_of_scales};
}

int check_scales(const unifur_nf4_scales* s) {
  UNIFUR_ARG(s != nullptr, "scales is NULL");
  if (s->kind == UNIFUR_NF4_SCALES_F32) {
    UNIFUR_ARG(s->absmax != nullptr, "F32 scales need absmax");
  } else if (s->kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED) {
    UNIFUR_ARG(s->dq_codes != nullptr && s->scale_of_scales != nullptr,
               "double-quantized scales need dq_codes and scale_of_scales");
  } else {
    return fail(UNIFUR_NF4_ERR_INVALID, "unknown scales kind " + std::to_string(s->kind));
  }
  return UNIFUR_NF4_OK;
}

bool aligned_to(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_weight(const unifur_nf4_weight* w, const char* name) {
  UNIFUR_ARG(w != nullptr, std::string(name) + " weight is NULL");
  UNIFUR_ARG(w->packed != nullptr, std::string(name) + " packed codes are NULL");
  UNIFUR_ARG(w->d_in > 0 && w->d_out > 0, std::string(name) + " has a zero dimension");
  UNIFUR_ARG(w->d_in <= 0x7fffffffu && w->d_out <= 0x7fffffffu, std::string(name) + " dimension exceeds 2^31-1");
  if (int r = check_scales(&w->scales)) return r;
  if (w->layout == UNIFUR_NF4_LAYOUT_ROW_MAJOR) return UNIFUR_NF4_OK;
  UNIFUR_ARG(w->layout == UNIFUR_NF4_LAYOUT_STRIPED,
             std::string(name) + " has unknown layout " + std::to_string(w->layout));
  UNIFUR_ARG(w->d_out % 64 == 0, std::string(name) + ": the striped layout needs d_out % 64 == 0");
  UNIFUR_ARG(aligned_to(w->packed, 8), std::string(name) + ": striped codes must be 8-byte aligned");
  UNIFUR_ARG(w->d_in * w->d_out / 2 < (1ull << 31), std::string(name) + ": striped weight over 2 GiB of codes");
  if (w->scales.kind == UNIFUR_NF4_SCALES_F32)
    UNIFUR_ARG(aligned_to(w->scales.absmax, 16), std::string(name) + ": striped absmax must be 16-byte aligned");
  else
    UNIFUR_ARG(aligned_to(w->scales.dq_codes, 4), std::string(name) + ": striped DQ codes must be 4-byte aligned");
  return UNIFUR_NF4_OK;
}

bool is_striped(const unifur_nf4_weight* w) { return w->layout == UNIFUR_NF4_LAYOUT_STRIPED; }

uint64_t scale_bytes(uint64_t num_blocks, int kind) {
  return kind == UNIFUR_NF4_SCALES_F32 ? 4 * num_blocks : num_blocks;
}

// ---------------------------------------------------------------- workspace --

struct WsCache {
  std::mutex mu;
  std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> buffers;
};

WsCache& ws_cache() {
  static WsCache* c = new WsCache();  // never destroyed: freeing at exit races the runtime teardown
  return *c;
}

// Internal workspace for (current device, stream), zero-filled when created.
// It only grows, and a buffer it outgrows is never freed: a graph captured
// from an earlier call may still hold its address, and a later replay must
// find it alive.  Under stream capture nothing is allocated, synchronized or
// filled: a call that would have to create or grow the buffer there fails
// with UNIFUR_NF4_ERR_WORKSPACE (make one eager call of the largest shape
// first, or pass a workspace).
int internal_workspace(size_t bytes, hipStream_t stream, void** out) {
  int dev = 0;
  UNIFUR_HIP(hipGetDevice(&dev));
  WsCache& c = ws_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  auto& slot = c.buffers[{dev, stream}];
  if (slot.second < bytes) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    UNIFUR_HIP(hipStreamIsCapturing(stream, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return fail(UNIFUR_NF4_ERR_WORKSPACE,
                  "the internal workspace of this stream holds " + std::to_string(slot.second) + " bytes, " +
                      std::to_string(bytes) + " needed, and the stream is capturing: make one eager call of "
                      "this shape first or pass a workspace");
    // grow at least twofold, so a rising sequence of shapes retires few
    // buffers; if the doubled size does not fit, try the size this call needs
    const size_t want = std::max<size_t>({bytes, size_t{1} << 20, 2 * slot.second});
    size_t sz = align_up(want);
    void* p = nullptr;
    if (hipMalloc(&p, sz) != hipSuccess) {
      (void)hipGetLastError();  // clear the failed allocation's error
      sz = align_up(std::max<size_t>(bytes, size_t{1} << 20));
      UNIFUR_HIP(hipMalloc(&p, sz));
    }
    UNIFUR_HIP(hipMemsetAsync(p, 0, sz, stream));
    slot = {p, sz};  // the outgrown buffer stays allocated until the process ends
  }
  *out = slot.first;
  return UNIFUR_NF4_OK;
}

int resolve_workspace(void* user, uint64_t user_bytes, size_t need, hipStream_t stream, void** out) {
  if (need == 0) {
    *out = user;
    return UNIFUR_NF4_OK;
  }
  if (user) {
    if (user_bytes < need)
      return fail(UNIFUR_NF4_ERR_WORKSPACE, "workspace of " + std::to_string(user_bytes) + " bytes, " +
                                                std::to_string(need) + " needed");
    *out = user;
    return UNIFUR_NF4_OK;
  }
  return internal_workspace(need, stream, out);
}

// Every workspace starts with a fixed region of split-K arrival counters.
// Only the GEMV's last-arrival logic writes it and it always leaves it zero,
// so it stays valid across calls of any shape and path; every other region
// (partials, dequantized weights, intermediates) is scratch carved after it.
constexpr size_t kCounterRegion = 64 << 10;
constexpr int kMaxCounters = (int)(kCounterRegion / sizeof(unsigned));

// Carves consecutive 256-byte-aligned regions out of one workspace.
// Shapes past any device: every element count a plan forms -- rows times a
// width, a weight's d_in x d_out, an MLP's middle -- stays at or below 2^48,
// so that no byte count derived from one (times an element size, a slab
// count, a rank of at most 64) wraps 64 bits.  Size queries answer
// UINT64_MAX for a shape past it and the calls refuse it.
constexpr uint64_t kMaxElements = 1ull << 48;
bool fits_elements(uint64_t a, uint64_t b) {
  uint64_t p = 0;
  return !__builtin_mul_overflow(a, b, &p) && p <= kMaxElements;
}
bool shape_fits(uint64_t rows, uint64_t d_in, uint64_t d_out) {
  return fits_elements(rows, d_in) && fits_elements(rows, d_out) && fits_elements(d_in, d_out);
}

struct Carver {
  size_t off = kCounterRegion;
  size_t take(size_t bytes) {
    size_t o = off;
    off += align_up(bytes);
    return o;
  }
};

// ------------------------------------------------------------- linear plans --

enum class LinearPath { kGemvStriped, kGemv, kSkinny, kMfma, kMfmaF32, kGeneric };

// The row-major GEMV needs whole 64-blocks per weight row (d_out % 64 == 0),
// 16-byte aligned code rows and a weight that 32-bit buffer offsets reach
// (under 2 GiB of codes, 4 G values).
bool gemv_layout_ok(uint64_t d_in, uint64_t d_out, const void* packed) {
  return d_out % 64 == 0 && aligned_to(packed, 16) && d_in * d_out / 2 < (1ull << 31);
}

struct LinearLayout {
  LinearPath path;
  bool expand;  // kMfma: bf16 weight expanded in the workspace + BLAS GEMM (else the fused kernel)
  GemvPlan gemv;
  StripedPlan striped, striped_tail;  // skinny: the plan of each launch (the last of several f32 launches)
  int splits = 1;  // kMfma without expand: d_in slabs of the fused kernel
  int tail = 1;    // ... or of only its last, partly filled round of tiles
  size_t partials, xa, lora_at, lora_bt, wt, blas, wf32, rm_codes, rm_scales, gemm_partials, total;
};

// Decode-sized batches (<= 4 rows) take a GEMV (the striped one for striped
// weights); bf16 batches up to 64 rows over a striped weight the skinny MFMA
// kernel; larger bf16 batches the prefill path: with `expand`, the weight
// (plus the LoRA update) expanded once to bf16 in the workspace and a BLAS
// GEMM, else the fused MFMA kernel that dequantizes W tiles in LDS (no
// weight-sized scratch); everything else the generic dequantize + f32
// matmul (a striped weight is first put back in row-major order in the
// workspace).
LinearLayout plan_linear(uint64_t rows, uint64_t d_in, uint64_t d_out, uint32_t lora_rank, const void* packed,
                         int x_dtype, const void* x, bool striped, int scale_kind, bool expand = true,
                         bool split = true) {
  LinearLayout L{};
  Carver c;
  const bool small = rows <= (uint64_t)kGemvMaxRows;
  const bool layout_ok = striped || gemv_layout_ok(d_in, d_out, packed);
  // bf16 batches past the GEMVs and the skinny kernel: the fused MFMA kernel
  // (X offsets under 2^31 bytes), or the expanded weight and the BLAS GEMM,
  // which address X with 64-bit offsets and so also take a batch past the
  // fused kernel's reach (more than 2 GiB of activations)
  const bool mfma_rows = !small && x_dtype == UNIFUR_NF4_BF16 && layout_ok && rows <= 0x7fffffffu;
  const bool mfma = mfma_rows && (gemm_supported((int)rows, (int)d_in, (int)d_out, x) ||
                                  (expand && aligned_to(x, 16) &&
                                   expand_supported((int)d_in, (int)d_out, (int)lora_rank)));
  // f32 activations: skinny launches of at most kSkinnyMaxRowsF32 rows each
  const bool xf32 = x_dtype == UNIFUR_NF4_F32;
  const uint64_t sk_rows = xf32 ? std::min<uint64_t>(rows, kSkinnyMaxRowsF32) : rows;
  const bool skinny = !small && striped && rows <= (uint64_t)kSkinnyMaxRows && d_in <= 0x7fffffffu &&
                      skinny_supported((int)sk_rows, (int)d_in, x, xf32) && d_out / 64 <= (uint64_t)kMaxCounters;
  if (small && striped) {
    L.path = LinearPath::kGemvStriped;
    const int n = (int)d_out;
    L.striped = plan_gemv_striped((int)rows, (int)d_in, &n, 1, false);
  } else if (skinny) {
    L.path = LinearPath::kSkinny;
    const int n = (int)d_out;
    L.striped = plan_skinny((int)sk_rows, (int)d_in, &n, 1, false);
    size_t part = skinny_partial_floats(L.striped, (int)sk_rows, n);
    if (rows > sk_rows) {  // the last f32 launch's own plan
      const int tail = (int)((rows - 1) % sk_rows + 1);
      L.striped_tail = plan_skinny(tail, (int)d_in, &n, 1, false);
      part = std::max(part, skinny_partial_floats(L.striped_tail, tail, n));
    }
    L.partials = c.take(part * sizeof(float));
  } else if (small && layout_ok && ceil_div_u64(d_out, 256) <= (uint64_t)kMaxCounters) {
    L.path = LinearPath::kGemv;
    const int n = (int)d_out;
    L.gemv = plan_gemv((int)rows, (int)d_in, &n, 1, false);
    L.partials = c.take(L.gemv.partial_count[0] * sizeof(float));
  } else if (mfma) {
    L.path = LinearPath::kMfma;
    L.expand = expand && expand_supported((int)d_in, (int)d_out, (int)lora_rank);
    if (L.expand) {
      L.wt = c.take(d_in * d_out * sizeof(uint16_t));
      L.blas = c.take(kBlasWorkspace);
    } else if (split && lora_rank == 0) {
      // the fused kernel over too few tiles splits d_in (f32 partials)
      L.splits = gemm_k_splits((int)rows, (int)d_in, (int)d_out);
      if (L.splits == 1) L.tail = gemm_tail_splits((int)rows, (int)d_in, (int)d_out);
      const int slabs = std::max(L.splits, L.tail);
      if (slabs > 1) L.gemm_partials = c.take((size_t)slabs * rows * d_out * sizeof(float));
    }
  } else if (xf32 && rows <= 0x7fffffffu && d_in <= 0x7fffffffu && d_out <= 0x7fffffffu && aligned_to(packed, 8) &&
             gemm_f32_mfma_supported((int)rows, (int)d_in, (int)d_out, (int)d_out, x)) {
    // f32 activations past the skinny kernel: the f32 MFMA kernel over W
    // tiles dequantized in LDS (no weight-sized scratch)
    L.path = LinearPath::kMfmaF32;
  } else {
    L.path = LinearPath::kGeneric;
    L.wf32 = c.take((size_t)d_in * d_out * sizeof(float));
    if (striped) {
      L.rm_codes = c.take(ceil_div_u64(d_in * d_out, 2));
      L.rm_scales = c.take(scale_bytes(ceil_div_u64(d_in * d_out, 64), scale_kind));
    }
  }
  if (L.path == LinearPath::kMfma && L.expand) {
    // the adapter is merged into the expanded weight
  } else if (L.path == LinearPath::kMfma && lora_rank) {
    // bf16 operands of the fused epilogue: xa [rows, pad], A^T [pad, d_in], B^T [d_out, pad]
    const size_t pad = (size_t)lora_pad((int)lora_rank);
    L.xa = c.take((size_t)rows * pad * 2);
    L.lora_at = c.take(pad * d_in * 2);
    L.lora_bt = c.take((size_t)d_out * pad * 2);
  } else if (L.path == LinearPath::kMfmaF32 && lora_rank) {
    // x A by the f32 MFMA row products ([rows][rank bucket] + their slab
    // partials), or the narrow kernel's [rows][rank]
    L.xa = c.take(std::max<size_t>((size_t)rows * lora_rank * sizeof(float),
                                   adapter_row_product_scratch_bytes((int)rows, (int)d_in, (int)lora_rank)));
  } else {
    L.xa = c.take((size_t)rows * lora_rank * sizeof(float));
  }
  L.total = c.off;
  return L;
}

template <typename T>
T* at(void* base, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

// A striped weight put back in row-major order into the workspace (the
// generic path's input); a row-major weight is returned as it is.
int row_major_view(const unifur_nf4_weight* w, void* ws, size_t codes_off, size_t scales_off, hipStream_t stream,
                   const uint8_t** packed, ScalesArg* scales) {
  *packed = w->packed;
  *scales = to_scales(w->scales);
  if (!is_striped(w)) return UNIFUR_NF4_OK;
  uint8_t* codes = at<uint8_t>(ws, codes_off);
  const bool dq = w->scales.kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED;
  UNIFUR_HIP(launch_stripe_codes(w->packed, codes, w->d_in, w->d_out, false, stream));
  void* sc = at<void>(ws, scales_off);
  UNIFUR_HIP(launch_stripe_scales(dq ? (const void*)w->scales.dq_codes : (const void*)w->scales.absmax, sc, w->d_in,
                                  w->d_out, dq, false, stream));
  *packed = codes;
  if (dq)
    scales->dq_codes = static_cast<const uint8_t*>(sc);
  else
    scales->absmax = static_cast<const float*>(sc);
  return UNIFUR_NF4_OK;
}

GemvWeight gemv_weight(const unifur_nf4_weight* w, void* y, bool y_bf16, unsigned* counters, float* partials) {
  GemvWeight g{};
  g.packed = w->packed;
  g.scales = to_scales(w->scales);
  g.d_out = (int)w->d_out;
  g.y = y;
  g.y_bf16 = y_bf16;
  g.counters = counters;
  g.partials = partials;
  return g;
}

// allow_expand == false keeps prefill batches on the fused MFMA kernel (no
// weight-sized scratch, no BLAS call), whatever the workspace size.
int run_linear(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w, const float* bias,
               const unifur_nf4_lora* lora, void* y, int y_dtype, void* workspace, uint64_t workspace_bytes,
               hipStream_t stream, bool allow_expand = true) {
  UNIFUR_ARG(valid_dtype(x_dtype) && valid_dtype(y_dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (int r = check_weight(w, "linear")) return r;
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x != nullptr && y != nullptr, "x or y is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  UNIFUR_ARG(shape_fits(rows, w->d_in, w->d_out), "linear: shape too large (an element count over 2^48)");
  const uint32_t rank = lora ? lora->rank : 0;
  if (lora) {
    UNIFUR_ARG(lora->a != nullptr && lora->b != nullptr, "lora factors are NULL");
    UNIFUR_ARG(rank >= 1 && rank <= 64, "lora rank must be in [1, 64]");
  }
  LinearLayout L = plan_linear(rows, w->d_in, w->d_out, rank, w->packed, x_dtype, x, is_striped(w), w->scales.kind,
                               allow_expand);
  if (L.path == LinearPath::kMfma && L.expand &&
      ((workspace && workspace_bytes < L.total) || !aligned_to(y, 16))) {
    // a workspace too small for the expanded weight (or an output the BLAS
    // kernels cannot take with 16-byte accesses): the fused kernel, or past
    // its reach the generic path
    LinearLayout lean =
        plan_linear(rows, w->d_in, w->d_out, rank, w->packed, x_dtype, x, is_striped(w), w->scales.kind, false);
    if (workspace && workspace_bytes < lean.total)  // without the split-K partials
      lean = plan_linear(rows, w->d_in, w->d_out, rank, w->packed, x_dtype, x, is_striped(w), w->scales.kind, false,
                         false);
    if (!workspace || workspace_bytes >= lean.total)
      L = lean;
    else if (!aligned_to(y, 16))
      return fail(UNIFUR_NF4_ERR_WORKSPACE, "linear: an output that is not 16-byte aligned needs " +
                                                std::to_string(lean.total) + " bytes of workspace here, got " +
                                                std::to_string(workspace_bytes));
  }
  if (L.path == LinearPath::kMfma && !L.expand && (L.splits > 1 || L.tail > 1) &&
      ((workspace && workspace_bytes < L.total) || !aligned_to(y, 16) || !aligned_to(bias, 16))) {
    // no room for the split-K partials (or an output or bias the reduction
    // cannot access four at a time): the fused kernel over whole d_in
    L = plan_linear(rows, w->d_in, w->d_out, rank, w->packed, x_dtype, x, is_striped(w), w->scales.kind, false,
                    false);
  }
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  const bool xbf = x_dtype == UNIFUR_NF4_BF16;
  const bool ybf = y_dtype == UNIFUR_NF4_BF16;
  float* xa = nullptr;
  if (L.path == LinearPath::kMfma && L.expand) {
    uint16_t* wt = at<uint16_t>(ws, L.wt);
    UNIFUR_HIP(launch_expand_bf16(w->packed, to_scales(w->scales), (int)w->d_in, (int)w->d_out, is_striped(w),
                                  lora ? lora->a : nullptr, lora ? lora->b : nullptr, (int)rank,
                                  lora ? lora->scaling : 0.0f, wt, stream));
    UNIFUR_HIP(blas_gemm_xwt(static_cast<const uint16_t*>(x), wt, bias, (int)rows, (int)w->d_out, (int)w->d_in, y,
                             ybf, at<void>(ws, L.blas), kBlasWorkspace, stream));
    return UNIFUR_NF4_OK;
  }
  if (L.path == LinearPath::kMfma) {
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    uint16_t *xa16 = nullptr, *bt16 = nullptr;
    if (lora) {
      xa16 = at<uint16_t>(ws, L.xa);
      bt16 = at<uint16_t>(ws, L.lora_bt);
      UNIFUR_HIP(launch_lora_operands(xb, lora->a, lora->b, (int)rows, (int)w->d_in, (int)w->d_out, (int)rank,
                                      lora->scaling, at<uint16_t>(ws, L.lora_at), bt16, xa16, stream));
    }
    UNIFUR_HIP(launch_gemm(xb, w->packed, to_scales(w->scales), (int)rows, (int)w->d_in, (int)w->d_out, bias, xa16,
                           bt16, (int)rank, y, ybf, is_striped(w), stream, L.splits,
                           L.splits > 1 || L.tail > 1 ? at<float>(ws, L.gemm_partials) : nullptr, L.tail));
    return UNIFUR_NF4_OK;
  }
  // f32 activations on MFMA: W tiles dequantized exactly in LDS; x A by the
  // f32 MFMA row products where they take the operands
  if (L.path == LinearPath::kMfmaF32) {
    int ld = (int)rank;
    if (lora) {
      xa = at<float>(ws, L.xa);
      if (adapter_row_product_supported(x, lora->a, (int)rows, (int)w->d_in, (int)rank)) {
        UNIFUR_HIP(launch_adapter_row_product(0, x, false, lora->a, (int)rows, (int)w->d_in, (int)rank, xa,
                                              at<unsigned>(ws, 0), kMaxCounters, stream));
        ld = adapter_row_product_ld((int)rank);
      } else {
        UNIFUR_HIP(launch_lora_xa(x, false, lora->a, (int)rows, (int)w->d_in, (int)rank, xa, stream));
      }
    }
    F32GemmArgs a{};
    a.x = static_cast<const float*>(x);
    a.packed = w->packed;
    a.scales = to_scales(w->scales);
    a.M = (int)rows;
    a.K = (int)w->d_in;
    a.N = (int)w->d_out;
    a.bias = bias;
    a.lora_xa = xa;
    a.lora_ld = ld;
    a.lora_b = lora ? lora->b : nullptr;
    a.lora_sbj = w->d_out;
    a.lora_sbn = 1;
    a.lora_rank = (int)rank;
    a.lora_scaling = lora ? lora->scaling : 0.0f;
    a.y = y;
    UNIFUR_HIP(launch_gemm_f32_mfma(a, w->scales.kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED, is_striped(w), false, ybf,
                                    stream));
    return UNIFUR_NF4_OK;
  }
  if (lora) {
    xa = at<float>(ws, L.xa);
    UNIFUR_HIP(launch_lora_xa(x, xbf, lora->a, (int)rows, (int)w->d_in, (int)rank, xa, stream));
  }
  if (L.path == LinearPath::kGemv || L.path == LinearPath::kGemvStriped || L.path == LinearPath::kSkinny) {
    GemvWeight gw = gemv_weight(w, y, ybf, at<unsigned>(ws, 0), at<float>(ws, L.partials));
    gw.bias = bias;
    gw.lora_xa = xa;
    gw.lora_b = lora ? lora->b : nullptr;
    gw.lora_rank = (int)rank;
    gw.lora_scaling = lora ? lora->scaling : 0.0f;
    if (L.path == LinearPath::kGemvStriped) {
      UNIFUR_HIP(launch_gemv_striped(L.striped, x, xbf, (int)rows, (int)w->d_in, &gw, 1, false, stream));
    } else if (L.path == LinearPath::kSkinny) {
      // bf16: one launch; f32: launches of up to kSkinnyMaxRowsF32 rows in
      // stream order (they take turns on the partials)
      const uint64_t step = xbf ? rows : (uint64_t)kSkinnyMaxRowsF32;
      const size_t xe = xbf ? 2 : 4, ye = ybf ? 2 : 4;
      for (uint64_t r0 = 0; r0 < rows; r0 += step) {
        const int n = (int)std::min<uint64_t>(step, rows - r0);
        GemvWeight g = gw;
        g.y = static_cast<char*>(y) + r0 * w->d_out * ye;
        if (xa) g.lora_xa = xa + r0 * rank;
        const StripedPlan& p = (r0 + step >= rows && r0 > 0) ? L.striped_tail : L.striped;
        UNIFUR_HIP(launch_skinny(p, static_cast<const char*>(x) + r0 * w->d_in * xe, !xbf, n, (int)w->d_in, &g, 1,
                                 false, stream));
      }
    } else {
      UNIFUR_HIP(launch_gemv(L.gemv, x, xbf, (int)rows, (int)w->d_in, &gw, 1, stream));
    }
    return UNIFUR_NF4_OK;
  }
  // Generic: the reference's own sequence -- dequantize the whole weight to
  // f32 (bit-exact), then an f32 matmul.
  const uint8_t* packed = nullptr;
  ScalesArg scales{};
  if (int r = row_major_view(w, ws, L.rm_codes, L.rm_scales, stream, &packed, &scales)) return r;
  float* wf = at<float>(ws, L.wf32);
  UNIFUR_HIP(launch_dequantize(packed, scales, (size_t)w->d_in * w->d_out, wf, false, u32_aligned(packed), stream));
  Epilogue e{bias, xa, lora ? lora->b : nullptr, (int)rank, lora ? lora->scaling : 0.0f, y, ybf};
  UNIFUR_HIP(launch_gemm_f32(x, xbf, wf, (int)rows, (int)w->d_in, (int)w->d_out, e, stream));
  return UNIFUR_NF4_OK;
}

// ------------------------------------------------------------- swiglu plans --

enum class MlpPath { kPairStriped, kStriped, kPairGemv, kGemv, kSkinny, kMfma, kGeneric };

struct MlpLayout {
  MlpPath path;
  bool expand;  // kMfma: each weight expanded to bf16 in turn + BLAS GEMMs (else the fused kernel)
  GemvPlan up_plan, down_plan;
  StripedPlan s_up, s_down;
  int split_up = 1, split_down = 1;  // kMfma without expand: d_in slabs of the fused kernel
  int tail_up = 1, tail_down = 1;    // ... or of only its last, partly filled round of tiles
  bool f32_mfma = false;             // kGeneric with f32 activations: the f32 MFMA kernel per linear
  size_t partials0, partials1, h, u, hb, wt, blas, wf32, rm_codes, rm_scales, gemm_partials, total;
};

constexpr int kFusedMlpMaxRows = 512;  // SwiGLU prefill: fused kernels up to this many rows

MlpLayout plan_mlp(uint64_t rows, uint64_t hidden, uint64_t inter, const unifur_nf4_weight* g,
                   const unifur_nf4_weight* u, const unifur_nf4_weight* d, int x_dtype, const void* x,
                   bool expand = true, bool split = true) {
  MlpLayout L{};
  Carver c;
  const bool all_striped = is_striped(g) && is_striped(u) && is_striped(d);
  const bool row_major_ok = !is_striped(g) && !is_striped(u) && !is_striped(d) &&
                            gemv_layout_ok(hidden, inter, g->packed) && gemv_layout_ok(hidden, inter, u->packed) &&
                            gemv_layout_ok(inter, hidden, d->packed) &&
                            ceil_div_u64(std::max(inter, hidden), 256) <= (uint64_t)kMaxCounters;
  const bool same_kind = g->scales.kind == u->scales.kind;
  const bool small = rows <= (uint64_t)kGemvMaxRows;
  const bool layouts_ok = all_striped || row_major_ok;
  // as for a single linear: the fused kernels within their X offsets' reach,
  // the expanded weights and BLAS GEMMs (64-bit offsets) past it
  const bool mfma_rows = !small && x_dtype == UNIFUR_NF4_BF16 && layouts_ok && rows <= 0x7fffffffu;
  const bool fused_ok =
      gemm_supported((int)rows, (int)hidden, (int)inter, x) &&
      gemm_supported((int)rows, (int)inter, (int)hidden, reinterpret_cast<const void*>(uintptr_t{256}));
  const bool mfma = mfma_rows && (fused_ok || (expand && rows > (uint64_t)kFusedMlpMaxRows && aligned_to(x, 16) &&
                                               expand_supported((int)hidden, (int)inter, 0) &&
                                               expand_supported((int)inter, (int)hidden, 0) &&
                                               2 * inter <= 0x7fffffffu));
  const int gi[2] = {(int)inter, (int)inter};
  const int hd = (int)hidden;
  // the skinny kernel for up to 64 bf16 (32 f32) rows; h lives 256-byte
  // aligned in the workspace
  const bool xf32 = x_dtype == UNIFUR_NF4_F32;
  const bool skinny = !small && all_striped && rows <= (uint64_t)kSkinnyMaxRows && hidden <= 0x7fffffffu &&
                      inter <= 0x7fffffffu && skinny_supported((int)rows, (int)hidden, x, xf32) &&
                      skinny_supported((int)rows, (int)inter, reinterpret_cast<const void*>(uintptr_t{256}), xf32) &&
                      std::max(inter, hidden) / 64 <= (uint64_t)kMaxCounters;
  if (skinny) {
    L.path = MlpPath::kSkinny;
    // same_kind: gate/up in one pair launch; else one launch each (the plan
    // of a single weight), both followed by down -- launches run in stream
    // order, so they take turns on the partials
    L.s_up = same_kind ? plan_skinny((int)rows, (int)hidden, gi, 2, true)
                       : plan_skinny((int)rows, (int)hidden, gi, 1, false);
    L.s_down = plan_skinny((int)rows, (int)inter, &hd, 1, false);
    const size_t up_part = skinny_partial_floats(L.s_up, (int)rows, (int)inter);
    L.partials0 = c.take(std::max(up_part, skinny_partial_floats(L.s_down, (int)rows, (int)hidden)) * sizeof(float));
    L.partials1 = c.take(up_part * sizeof(float));
    L.hb = c.take((size_t)rows * inter * sizeof(uint16_t));
    if (!same_kind || xf32) L.h = c.take((size_t)rows * inter * sizeof(float));  // f32 x: the middle stays f32
    if (!same_kind) L.u = c.take((size_t)rows * inter * sizeof(float));
  } else if (small && all_striped) {
    L.path = rows <= (uint64_t)kGemvPairMaxRows && same_kind ? MlpPath::kPairStriped : MlpPath::kStriped;
    L.s_up = plan_gemv_striped((int)rows, (int)hidden, gi, 2, L.path == MlpPath::kPairStriped);
    L.s_down = plan_gemv_striped((int)rows, (int)inter, &hd, 1, false);
    L.h = c.take((size_t)rows * inter * sizeof(float));
    L.u = L.path == MlpPath::kStriped ? c.take((size_t)rows * inter * sizeof(float)) : 0;
  } else if (small && row_major_ok) {
    L.path = rows <= (uint64_t)kGemvPairMaxRows && same_kind ? MlpPath::kPairGemv : MlpPath::kGemv;
    L.up_plan = plan_gemv((int)rows, (int)hidden, gi, 2, L.path == MlpPath::kPairGemv);
    L.down_plan = plan_gemv((int)rows, (int)inter, &hd, 1, false);
    L.partials0 = c.take(std::max(L.up_plan.partial_count[0], L.down_plan.partial_count[0]) * sizeof(float));
    L.partials1 = c.take(L.up_plan.partial_count[1] * sizeof(float));
    L.h = c.take((size_t)rows * inter * sizeof(float));
    L.u = L.path == MlpPath::kGemv ? c.take((size_t)rows * inter * sizeof(float)) : 0;
  } else if (mfma) {
    L.path = MlpPath::kMfma;
    // up to 512 rows the fused kernels with split-K win (7B-shaped MLP: 149
    // against 181.5 us at 256 rows, 229.6 against 238 us at 512); above, the
    // weights expanded once and the BLAS GEMMs
    L.expand = expand && rows > (uint64_t)kFusedMlpMaxRows && expand_supported((int)hidden, (int)inter, 0) &&
               expand_supported((int)inter, (int)hidden, 0) && 2 * inter <= 0x7fffffffu;
    if (L.expand) {
      // gate and up expanded side by side ([2 inter][hidden]: one GEMM with
      // f32 outputs [rows][2 inter], so silu(g) * u is rounded to bf16 once,
      // as on the fused path), then down into the same buffer
      L.wt = c.take(2 * hidden * inter * sizeof(uint16_t));
      L.blas = c.take(kBlasWorkspace);
      L.h = c.take((size_t)rows * 2 * inter * sizeof(float));
      L.hb = c.take((size_t)rows * inter * sizeof(uint16_t));
    } else {
      // gate and up of one scale kind: one pair launch storing bf16
      // silu(g) * u; else one launch each (f32 outputs) and the elementwise
      // kernel
      if (!same_kind) {
        L.h = c.take((size_t)rows * inter * sizeof(float));
        L.u = c.take((size_t)rows * inter * sizeof(float));
      }
      L.hb = c.take((size_t)rows * inter * sizeof(uint16_t));
      if (split) {  // the fused kernel splits d_in where its grid would leave CUs idle (f32 partials)
        L.split_up = gemm_k_splits((int)rows, (int)hidden, (int)inter, same_kind);
        L.split_down = gemm_k_splits((int)rows, (int)inter, (int)hidden);
        if (L.split_up == 1) L.tail_up = gemm_tail_splits((int)rows, (int)hidden, (int)inter, same_kind);
        if (L.split_down == 1) L.tail_down = gemm_tail_splits((int)rows, (int)inter, (int)hidden);
        const size_t up_slabs = (size_t)std::max(L.split_up, L.tail_up), down_slabs = std::max(L.split_down, L.tail_down);
        const size_t part = std::max(up_slabs > 1 ? up_slabs * rows * inter * (same_kind ? 2 : 1) : 0,
                                     down_slabs > 1 ? down_slabs * rows * hidden : 0);
        if (part) L.gemm_partials = c.take(part * sizeof(float));
      }
    }
  } else {
    L.path = MlpPath::kGeneric;
    // f32 activations: the three linears on the f32 MFMA kernel (no f32 weight copy)
    L.f32_mfma = x_dtype == UNIFUR_NF4_F32 && rows <= 0x7fffffffu && hidden <= 0x7fffffffu && inter <= 0x7fffffffu &&
                 hidden % 64 == 0 && aligned_to(g->packed, 8) && aligned_to(u->packed, 8) && aligned_to(d->packed, 8) && gemm_f32_mfma_supported((int)rows, (int)hidden, (int)inter, (int)inter, x) &&
                 gemm_f32_mfma_supported((int)rows, (int)inter, (int)hidden, (int)hidden,
                                         reinterpret_cast<const void*>(uintptr_t{256}));
    L.h = c.take((size_t)rows * inter * sizeof(float));
    L.u = c.take((size_t)rows * inter * sizeof(float));
    if (L.f32_mfma) {
      L.total = c.off;
      return L;
    }
    L.wf32 = c.take((size_t)hidden * inter * sizeof(float));
    if (is_striped(g) || is_striped(u) || is_striped(d)) {
      L.rm_codes = c.take(ceil_div_u64(hidden * inter, 2));
      L.rm_scales = c.take(4 * ceil_div_u64(hidden * inter, 64));
    }
  }
  L.total = c.off;
  return L;
}

int run_swiglu(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* gate, const unifur_nf4_weight* up,
               const unifur_nf4_weight* down, void* y, int y_dtype, void* workspace, uint64_t workspace_bytes,
               hipStream_t stream) {
  UNIFUR_ARG(valid_dtype(x_dtype) && valid_dtype(y_dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (int r = check_weight(gate, "gate")) return r;
  if (int r = check_weight(up, "up")) return r;
  if (int r = check_weight(down, "down")) return r;
  const uint64_t hidden = gate->d_in, inter = gate->d_out;
  UNIFUR_ARG(up->d_in == hidden && up->d_out == inter, "up must be [hidden, intermediate] like gate");
  UNIFUR_ARG(down->d_in == inter && down->d_out == hidden, "down must be [intermediate, hidden]");
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x != nullptr && y != nullptr, "x or y is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  UNIFUR_ARG(shape_fits(rows, hidden, inter), "swiglu: shape too large (an element count over 2^48)");
  MlpLayout L = plan_mlp(rows, hidden, inter, gate, up, down, x_dtype, x);
  if (L.path == MlpPath::kMfma && L.expand && ((workspace && workspace_bytes < L.total) || !aligned_to(y, 16))) {
    // a workspace too small for an expanded weight, or an output the BLAS
    // kernels cannot take with 16-byte accesses: the fused kernel
    MlpLayout lean = plan_mlp(rows, hidden, inter, gate, up, down, x_dtype, x, false);
    if (workspace && workspace_bytes < lean.total)  // without the split-K partials
      lean = plan_mlp(rows, hidden, inter, gate, up, down, x_dtype, x, false, false);
    if (workspace_bytes >= lean.total || !workspace)
      L = lean;
    else if (!aligned_to(y, 16))
      return fail(UNIFUR_NF4_ERR_WORKSPACE, "swiglu: an output that is not 16-byte aligned needs " +
                                                std::to_string(lean.total) + " bytes of workspace here, got " +
                                                std::to_string(workspace_bytes));
  }
  if (L.path == MlpPath::kMfma && !L.expand && L.gemm_partials &&
      ((workspace && workspace_bytes < L.total) || !aligned_to(y, 16)))
    L = plan_mlp(rows, hidden, inter, gate, up, down, x_dtype, x, false, false);  // without split-K
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  const bool xbf = x_dtype == UNIFUR_NF4_BF16;
  const bool ybf = y_dtype == UNIFUR_NF4_BF16;
  float* h = at<float>(ws, L.h);
  unsigned* cnt = at<unsigned>(ws, 0);
  switch (L.path) {
    case MlpPath::kPairStriped: {
      GemvWeight gw[2] = {gemv_weight(gate, h, false, cnt, nullptr), gemv_weight(up, nullptr, false, cnt, nullptr)};
      UNIFUR_HIP(launch_gemv_striped(L.s_up, x, xbf, (int)rows, (int)hidden, gw, 2, true, stream));
      GemvWeight dw = gemv_weight(down, y, ybf, cnt, nullptr);
      UNIFUR_HIP(launch_gemv_striped(L.s_down, h, false, (int)rows, (int)inter, &dw, 1, false, stream));
      return UNIFUR_NF4_OK;
    }
    case MlpPath::kStriped: {
      float* u = at<float>(ws, L.u);
      // gate and up in one launch (two weights over the same x) when their
      // scales are of one kind, else one launch each
      GemvWeight gw[2] = {gemv_weight(gate, h, false, cnt, nullptr), gemv_weight(up, u, false, cnt, nullptr)};
      if (gate->scales.kind == up->scales.kind) {
        UNIFUR_HIP(launch_gemv_striped(L.s_up, x, xbf, (int)rows, (int)hidden, gw, 2, false, stream));
      } else {
        const StripedPlan one = plan_gemv_striped((int)rows, (int)hidden, &gw[0].d_out, 1, false);
        UNIFUR_HIP(launch_gemv_striped(one, x, xbf, (int)rows, (int)hidden, &gw[0], 1, false, stream));
        UNIFUR_HIP(launch_gemv_striped(one, x, xbf, (int)rows, (int)hidden, &gw[1], 1, false, stream));
      }
      UNIFUR_HIP(launch_silu_mul(h, u, (size_t)rows * inter, h, stream));
      GemvWeight dw = gemv_weight(down, y, ybf, cnt, nullptr);
      UNIFUR_HIP(launch_gemv_striped(L.s_down, h, false, (int)rows, (int)inter, &dw, 1, false, stream));
      return UNIFUR_NF4_OK;
    }
    case MlpPath::kPairGemv:
    case MlpPath::kGemv: {
      float* p0 = at<float>(ws, L.partials0);
      float* p1 = at<float>(ws, L.partials1);
      if (L.path == MlpPath::kPairGemv) {
        GemvWeight gw[2] = {gemv_weight(gate, h, false, cnt, p0), gemv_weight(up, nullptr, false, cnt, p1)};
        UNIFUR_HIP(launch_gemv(L.up_plan, x, xbf, (int)rows, (int)hidden, gw, 2, stream));
      } else {
        float* u = at<float>(ws, L.u);
        GemvWeight g1 = gemv_weight(gate, h, false, cnt, p0);
        UNIFUR_HIP(launch_gemv(plan_gemv((int)rows, (int)hidden, &g1.d_out, 1, false), x, xbf, (int)rows,
                               (int)hidden, &g1, 1, stream));
        GemvWeight g2 = gemv_weight(up, u, false, cnt, p0);
        UNIFUR_HIP(launch_gemv(plan_gemv((int)rows, (int)hidden, &g2.d_out, 1, false), x, xbf, (int)rows,
                               (int)hidden, &g2, 1, stream));
        UNIFUR_HIP(launch_silu_mul(h, u, (size_t)rows * inter, h, stream));
      }
      GemvWeight dw = gemv_weight(down, y, ybf, cnt, p0);
      UNIFUR_HIP(launch_gemv(L.down_plan, h, false, (int)rows, (int)inter, &dw, 1, stream));
      return UNIFUR_NF4_OK;
    }
    case MlpPath::kSkinny: {
      // gate and up in one pass storing silu(g) * u -- bf16 for bf16 x, f32
      // for f32 x -- (two passes and the elementwise kernel when their scales
      // differ in kind), then down over that middle
      const bool xf = !xbf;
      uint16_t* hb = at<uint16_t>(ws, L.hb);
      void* mid = xf ? static_cast<void*>(h) : static_cast<void*>(hb);
      float* p0 = at<float>(ws, L.partials0);
      float* p1 = at<float>(ws, L.partials1);
      if (gate->scales.kind == up->scales.kind) {
        GemvWeight gw[2] = {gemv_weight(gate, mid, !xf, cnt, p0), gemv_weight(up, nullptr, !xf, cnt, p1)};
        UNIFUR_HIP(launch_skinny(L.s_up, x, xf, (int)rows, (int)hidden, gw, 2, true, stream));
      } else {
        float* u = at<float>(ws, L.u);
        GemvWeight gw[2] = {gemv_weight(gate, h, false, cnt, p0), gemv_weight(up, u, false, cnt, p0)};
        UNIFUR_HIP(launch_skinny(L.s_up, x, xf, (int)rows, (int)hidden, &gw[0], 1, false, stream));
        UNIFUR_HIP(launch_skinny(L.s_up, x, xf, (int)rows, (int)hidden, &gw[1], 1, false, stream));
        if (xf)
          UNIFUR_HIP(launch_silu_mul(h, u, (size_t)rows * inter, h, stream));
        else
          UNIFUR_HIP(launch_silu_mul_bf16(h, u, (size_t)rows * inter, hb, stream));
      }
      GemvWeight dw = gemv_weight(down, y, ybf, cnt, p0);
      UNIFUR_HIP(launch_skinny(L.s_down, mid, xf, (int)rows, (int)inter, &dw, 1, false, stream));
      return UNIFUR_NF4_OK;
    }
    case MlpPath::kMfma: {
      // gate and up (f32 out), silu(g) * u rounded to bf16 once, then down:
      // each weight expanded to bf16 in turn and a BLAS GEMM, or the fused
      // kernel -- both paths round the same intermediates.
      const uint16_t* xb = static_cast<const uint16_t*>(x);
      float* u = at<float>(ws, L.u);
      uint16_t* hb = at<uint16_t>(ws, L.hb);
      if (L.expand) {
        uint16_t* wt = at<uint16_t>(ws, L.wt);
        float* gu = at<float>(ws, L.h);
        void* bw = at<void>(ws, L.blas);
        const int hd = (int)hidden, in = (int)inter, m = (int)rows;
        UNIFUR_HIP(launch_expand_bf16(gate->packed, to_scales(gate->scales), hd, in, is_striped(gate), nullptr,
                                      nullptr, 0, 0.0f, wt, stream));
        UNIFUR_HIP(launch_expand_bf16(up->packed, to_scales(up->scales), hd, in, is_striped(up), nullptr, nullptr, 0,
                                      0.0f, wt + (size_t)in * hd, stream));
        UNIFUR_HIP(blas_gemm_xwt(xb, wt, nullptr, m, 2 * in, hd, gu, false, bw, kBlasWorkspace, stream));
        UNIFUR_HIP(launch_silu_mul_rows_bf16(gu, true, (size_t)rows, (size_t)inter, hb, stream));
        UNIFUR_HIP(launch_expand_bf16(down->packed, to_scales(down->scales), in, hd, is_striped(down), nullptr,
                                      nullptr, 0, 0.0f, wt, stream));
        UNIFUR_HIP(blas_gemm_xwt(hb, wt, nullptr, m, hd, in, y, ybf, bw, kBlasWorkspace, stream));
        return UNIFUR_NF4_OK;
      }
      float* gp = L.gemm_partials ? at<float>(ws, L.gemm_partials) : nullptr;
      if (gate->scales.kind == up->scales.kind) {
        UNIFUR_HIP(launch_gemm_pair(xb, gate->packed, to_scales(gate->scales), up->packed, to_scales(up->scales),
                                    (int)rows, (int)hidden, (int)inter, hb, is_striped(gate), stream, L.split_up, gp,
                                    L.tail_up));
      } else {
        UNIFUR_HIP(launch_gemm(xb, gate->packed, to_scales(gate->scales), (int)rows, (int)hidden, (int)inter, nullptr,
                               nullptr, nullptr, 0, h, false, is_striped(gate), stream, L.split_up, gp, L.tail_up));
        UNIFUR_HIP(launch_gemm(xb, up->packed, to_scales(up->scales), (int)rows, (int)hidden, (int)inter, nullptr,
                               nullptr, nullptr, 0, u, false, is_striped(up), stream, L.split_up, gp, L.tail_up));
        UNIFUR_HIP(launch_silu_mul_bf16(h, u, (size_t)rows * inter, hb, stream));
      }
      UNIFUR_HIP(launch_gemm(hb, down->packed, to_scales(down->scales), (int)rows, (int)inter, (int)hidden, nullptr,
                             nullptr, nullptr, 0, y, ybf, is_striped(down), stream, L.split_down, gp, L.tail_down));
      return UNIFUR_NF4_OK;
    }
    case MlpPath::kGeneric:
      break;
  }
  if (L.f32_mfma) {  // f32 activations: three f32 MFMA launches and the elementwise middle
    float* u = at<float>(ws, L.u);
    const unifur_nf4_weight* ws3[3] = {gate, up, down};
    void* outs[3] = {h, u, y};
    for (int i = 0; i < 3; ++i) {
      const unifur_nf4_weight* w = ws3[i];
      F32GemmArgs a{};
      a.x = i < 2 ? static_cast<const float*>(x) : h;
      a.packed = w->packed;
      a.scales = to_scales(w->scales);
      a.M = (int)rows;
      a.K = (int)w->d_in;
      a.N = (int)w->d_out;
      a.y = outs[i];
      UNIFUR_HIP(launch_gemm_f32_mfma(a, w->scales.kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED, is_striped(w), false,
                                      i == 2 && ybf, stream));
      if (i == 1) UNIFUR_HIP(launch_silu_mul(h, u, (size_t)rows * inter, h, stream));
    }
    return UNIFUR_NF4_OK;
  }
  // Generic: three dequantize + f32 matmul linears and the elementwise middle.
  float* wf = at<float>(ws, L.wf32);
  float* u = at<float>(ws, L.u);
  const Epilogue none{};
  Epilogue eg = none, eu = none, ed = none;
  eg.y = h;
  eu.y = u;
  ed.y = y;
  ed.y_bf16 = ybf;
  const unifur_nf4_weight* ws3[3] = {gate, up, down};
  const Epilogue* es[3] = {&eg, &eu, &ed};
  for (int i = 0; i < 3; ++i) {
    const unifur_nf4_weight* w = ws3[i];
    const uint8_t* packed = nullptr;
    ScalesArg scales{};
    if (int r = row_major_view(w, ws, L.rm_codes, L.rm_scales, stream, &packed, &scales)) return r;
    UNIFUR_HIP(launch_dequantize(packed, scales, w->d_in * w->d_out, wf, false, u32_aligned(packed), stream));
    if (i < 2) {
      UNIFUR_HIP(launch_gemm_f32(x, xbf, wf, (int)rows, (int)hidden, (int)inter, *es[i], stream));
      if (i == 1) UNIFUR_HIP(launch_silu_mul(h, u, (size_t)rows * inter, h, stream));
    } else {
      UNIFUR_HIP(launch_gemm_f32(h, false, wf, (int)rows, (int)inter, (int)hidden, *es[i], stream));
    }
  }
  return UNIFUR_NF4_OK;
}

uint64_t swiglu_workspace(uint64_t rows, uint64_t hidden, uint64_t intermediate, int x_dtype, bool expand,
                          bool split = true) {
  if (rows == 0 || hidden == 0 || intermediate == 0) return 0;
  if (rows > 0x7fffffffu || !shape_fits(rows, hidden, intermediate)) return UINT64_MAX;
  const uint8_t* p = reinterpret_cast<const uint8_t*>(uintptr_t{256});
  uint64_t need = 0;
  for (int striped = 0; striped < 2; ++striped) {
    if (striped && (hidden % 64 != 0 || intermediate % 64 != 0)) continue;
    for (int kind = 0; kind < 4; ++kind) {  // gate and up scale kinds, alike or not
      unifur_nf4_weight g{p, {kind & 1, (const float*)p, p, (const float*)p}, hidden, intermediate,
                          striped ? UNIFUR_NF4_LAYOUT_STRIPED : UNIFUR_NF4_LAYOUT_ROW_MAJOR};
      unifur_nf4_weight u = g;
      u.scales.kind = kind >> 1;
      unifur_nf4_weight d = g;
      d.d_in = intermediate;
      d.d_out = hidden;
      need = std::max<uint64_t>(need,
                                plan_mlp(rows, hidden, intermediate, &g, &u, &d, x_dtype, p, expand, split).total);
    }
  }
  return need;
}


// -------------------------------------------------------- concurrent branch --

// A second stream per (device, caller stream) for work that is independent of
// the caller stream's next launches: forked from the caller stream and joined
// back into it with events, which a graph capture records as a fork and a
// join.  It is created on first use outside capture; a call under capture
// that finds none runs everything on the caller stream.  Default priority,
// like every stream here.
struct Branch {
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

struct BranchCache {
  std::mutex mu;
  std::map<std::pair<int, hipStream_t>, Branch> branches;
};

BranchCache& branch_cache() {
  static BranchCache* c = new BranchCache();  // never destroyed, like the workspaces
  return *c;
}

Branch branch_for(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return {};
  BranchCache& c = branch_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  const auto it = c.branches.find({dev, stream});
  if (it != c.branches.end()) return it->second;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return {};
  Branch b;
  if (hipStreamCreateWithFlags(&b.side, hipStreamNonBlocking) != hipSuccess) return {};
  if (hipEventCreateWithFlags(&b.fork, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&b.join, hipEventDisableTiming) != hipSuccess) {
    if (b.fork) (void)hipEventDestroy(b.fork);
    (void)hipStreamDestroy(b.side);
    return {};
  }
  c.branches[{dev, stream}] = b;
  return b;
}

// ------------------------------------------------------------ backward -----

// dX through the expanded bf16 weight and the BLAS GEMM (bf16 dY), or the
// generic dequantize (+ merge) and f32 GEMM; the adapter gradients through
// x A, dY B^T and two row reductions.
struct BackwardLayout {
  bool blas, fused;
  int splits;  // fused dX: d_out slabs (1: none)
  bool mfma_f32;  // f32 dY: the f32 MFMA kernel over W's rows (dY B^T in dy_bt when there is an adapter)
  size_t dy_bt;
  size_t wt, blas_ws, wf32, rm_codes, rm_scales, lora_at, lora_bt, lora_xa, dx_partials, grads, xa, u, partials, total;
};

// dX paths: the weight expanded to bf16 once and a BLAS GEMM (blas), the
// fused NF4 MFMA kernel over the striped weight's rows (fused: only the
// adapter's bf16 operands, or split-K partials, as scratch), or the generic
// f32 dequantize + GEMM.  allow_blas = false picks the fused kernel where it
// applies (a workspace too small for the expanded weight); allow_split =
// false leaves out its split-K partials.
BackwardLayout plan_backward(uint64_t rows, uint64_t d_in, uint64_t d_out, uint32_t rank, int dy_dtype, bool want_dx,
                             bool want_grads, bool striped, int scale_kind, bool aligned, bool allow_blas = true,
                             bool allow_split = true, bool codes_aligned = true) {
  BackwardLayout L{};
  L.splits = 1;
  Carver c;
  if (want_dx) {
    const bool sizes = rows <= 0x7fffffffu && d_in <= 0x7fffffffu && d_out <= 0x7fffffffu;
    const bool bf = dy_dtype == UNIFUR_NF4_BF16 && aligned && sizes;
    L.blas = allow_blas && bf && expand_supported((int)d_in, (int)d_out, (int)rank);
    // the dX GEMM's shape: M = rows, reduction d_out, outputs d_in
    L.fused = !L.blas && bf && striped && rank <= 64 && rows >= 1 &&
              gemm_supported((int)rows, (int)d_out, (int)d_in, reinterpret_cast<const void*>(uintptr_t{256}));
    if (L.blas) {
      L.wt = c.take(d_in * d_out * sizeof(uint16_t));
      L.blas_ws = c.take(kBlasWorkspace);
    } else if (L.fused) {
      if (rank) {
        const uint64_t pad = (uint64_t)lora_pad((int)rank);
        L.lora_at = c.take(pad * d_out * sizeof(uint16_t));
        L.lora_bt = c.take(d_in * pad * sizeof(uint16_t));
        L.lora_xa = c.take(rows * pad * sizeof(uint16_t));
      } else if (allow_split) {
        L.splits = gemm_k_splits((int)rows, (int)d_out, (int)d_in);
        if (L.splits > 1) L.dx_partials = c.take((size_t)L.splits * rows * d_in * sizeof(float));
      }
    } else if (dy_dtype == UNIFUR_NF4_F32 && aligned && codes_aligned && sizes && d_out % 64 == 0 &&
               gemm_f32_mfma_supported((int)rows, (int)d_out, (int)d_in, (int)d_out,
                                       reinterpret_cast<const void*>(uintptr_t{256}))) {
      // f32 dY: dX on the f32 MFMA kernel with W's rows as its outputs
      L.mfma_f32 = true;
      if (rank)
        L.dy_bt = c.take(std::max<size_t>((size_t)rows * rank * sizeof(float),
                                          adapter_row_product_scratch_bytes((int)rows, (int)d_out, (int)rank)));
    } else {
      L.wf32 = c.take(d_in * d_out * sizeof(float));
      if (striped) {
        L.rm_codes = c.take(ceil_div_u64(d_in * d_out, 2));
        L.rm_scales = c.take(scale_bytes(ceil_div_u64(d_in * d_out, 64), scale_kind));
      }
    }
  }
  if (want_grads && rank) {
    // one region for the MFMA kernels' scratch or, for operands they do not
    // take, the narrow kernels' x A, dY B^T and slab partials
    const int m = (int)std::min<uint64_t>(rows, 0x7fffffffu);
    const int k = (int)std::min<uint64_t>(d_in, 0x7fffffffu), n = (int)std::min<uint64_t>(d_out, 0x7fffffffu);
    Carver g;
    g.off = 0;
    L.xa = g.take((size_t)rows * rank * sizeof(float));
    L.u = g.take((size_t)rows * rank * sizeof(float));
    const size_t p_mm = (size_t)std::max(narrow_mm_slabs(m, k), narrow_mm_slabs(m, n)) * rows * rank;
    const size_t p_atb = std::max((size_t)narrow_atb_slabs(m, n) * d_out, (size_t)narrow_atb_slabs(m, k) * d_in) * rank;
    L.partials = g.take(std::max(p_mm, p_atb) * sizeof(float));
    L.grads = c.take(std::max<size_t>(g.off, adapter_grads_scratch_bytes(m, k, n, (int)rank)));
    L.xa += L.grads;
    L.u += L.grads;
    L.partials += L.grads;
  }
  L.total = c.off;
  return L;
}

int run_backward(const void* dy, int dy_dtype, uint64_t rows, const unifur_nf4_weight* w, const unifur_nf4_lora* lora,
                 const void* x, int x_dtype, void* dx, int dx_dtype, float* grad_a, float* grad_b, void* workspace,
                 uint64_t workspace_bytes, hipStream_t stream) {
  UNIFUR_ARG(valid_dtype(dy_dtype) && valid_dtype(dx_dtype) && valid_dtype(x_dtype),
             "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (int r = check_weight(w, "linear_backward")) return r;
  const uint32_t rank = lora ? lora->rank : 0;
  if (lora) {
    UNIFUR_ARG(lora->a != nullptr && lora->b != nullptr, "lora factors are NULL");
    UNIFUR_ARG(rank >= 1 && rank <= 64, "lora rank must be in [1, 64]");
  }
  const bool want_dx = dx != nullptr;
  const bool want_grads = lora && (grad_a || grad_b);
  UNIFUR_ARG(!(grad_a || grad_b) || lora, "adapter gradients need the adapter");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  UNIFUR_ARG(rows == 0 || dy != nullptr, "dy is NULL");
  UNIFUR_ARG(!want_grads || rows == 0 || x != nullptr, "adapter gradients need x");
  const uint64_t K = w->d_in, N = w->d_out;
  UNIFUR_ARG(K <= 0x7fffffffu && N <= 0x7fffffffu, "weight too large");
  UNIFUR_ARG(shape_fits(rows, K, N), "linear_backward: shape too large (an element count over 2^48)");
  const bool aligned = aligned_to(dy, 16) && aligned_to(dx, 16);
  BackwardLayout L = plan_backward(rows, K, N, rank, dy_dtype, want_dx && rows > 0, want_grads, is_striped(w),
                                   w->scales.kind, aligned, true, true, aligned_to(w->packed, 8));
  if (L.blas && workspace && workspace_bytes < L.total) {
    // a workspace too small for the expanded weight: the fused dX kernel,
    // with its split-K partials if they fit
    BackwardLayout lean = plan_backward(rows, K, N, rank, dy_dtype, true, want_grads, is_striped(w), w->scales.kind,
                                        aligned, false);
    if (lean.fused && workspace_bytes < lean.total)
      lean = plan_backward(rows, K, N, rank, dy_dtype, true, want_grads, is_striped(w), w->scales.kind, aligned,
                           false, false);
    if (lean.fused && workspace_bytes >= lean.total) L = lean;
  }
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  const bool dybf = dy_dtype == UNIFUR_NF4_BF16, xbf = x_dtype == UNIFUR_NF4_BF16;
  const int m = (int)rows, k = (int)K, n = (int)N;
  const bool mfma_grads = want_grads && adapter_grads_supported(x, dy, lora->b, m, k, n, (int)rank);
  const auto grads_on = [&](hipStream_t s) -> hipError_t {
    return launch_adapter_grads(x, xbf, dy, dybf, lora->a, lora->b, m, k, n, (int)rank, lora->scaling, grad_a,
                                grad_b, at<void>(ws, L.grads), static_cast<unsigned*>(ws), kMaxCounters, s);
  };
  // With both dX (expand + BLAS GEMM) and the MFMA adapter gradients to do,
  // the gradients run on a branch stream beside the dX GEMM: they read x and
  // dY and write their own scratch, counters and outputs, disjoint from dX's.
  bool grads_done = false;
  if (want_dx && rows > 0) {
    // dX = dY (W + scaling A B)^T = dY W^T + ((dY scaling) B^T) A^T
    if (L.blas) {
      // E = bf16(W + scaling A B) in W's own [d_in][d_out] orientation, so
      // that dX = dY E^T is the forward's TN product
      uint16_t* e_rows = at<uint16_t>(ws, L.wt);
      const Branch br = mfma_grads ? branch_for(stream) : Branch{};
      bool forked = false;
      const auto fork = [&]() -> hipError_t {
        hipError_t e = hipEventRecord(br.fork, stream);
        if (e != hipSuccess) return e;
        if ((e = hipStreamWaitEvent(br.side, br.fork, 0)) != hipSuccess) return e;
        forked = true;
        e = grads_on(br.side);
        const hipError_t j = hipEventRecord(br.join, br.side);  // recorded even when the launch failed
        return e != hipSuccess ? e : j;
      };
      hipError_t e = launch_expand_rows_bf16(w->packed, to_scales(w->scales), k, n, is_striped(w),
                                             lora ? lora->a : nullptr, lora ? lora->b : nullptr, (int)rank,
                                             lora ? lora->scaling : 0.0f, e_rows, stream);
      // the gradients beside the GEMM, not the memory-bound expand; on a
      // shape's first call the GEMM's kernel is chosen by timing candidates,
      // so the gradients wait and run after it instead of contending
      if (e == hipSuccess && br.side && blas_gemm_xwt_tuned(m, k, n, dx_dtype == UNIFUR_NF4_BF16)) e = fork();
      if (e == hipSuccess)
        e = blas_gemm_xwt(static_cast<const uint16_t*>(dy), e_rows, nullptr, m, k, n, dx,
                          dx_dtype == UNIFUR_NF4_BF16, at<void>(ws, L.blas_ws), kBlasWorkspace, stream);
      if (forked) {  // every exit after a fork joins it first
        const hipError_t jn = hipStreamWaitEvent(stream, br.join, 0);
        if (e == hipSuccess) e = jn;
      }
      grads_done = forked;
      UNIFUR_HIP(e);
    } else if (L.fused) {
      const uint16_t* dyb = static_cast<const uint16_t*>(dy);
      uint16_t *xa16 = nullptr, *bt16 = nullptr;
      if (lora) {
        xa16 = at<uint16_t>(ws, L.lora_xa);
        bt16 = at<uint16_t>(ws, L.lora_bt);
        UNIFUR_HIP(launch_lora_operands_dx(dyb, lora->a, lora->b, m, k, n, (int)rank, lora->scaling,
                                           at<uint16_t>(ws, L.lora_at), bt16, xa16, stream));
      }
      UNIFUR_HIP(launch_gemm_dx(dyb, w->packed, to_scales(w->scales), m, k, n, xa16, bt16, (int)rank, dx,
                                dx_dtype == UNIFUR_NF4_BF16, stream, L.splits,
                                L.splits > 1 ? at<float>(ws, L.dx_partials) : nullptr));
    } else if (L.mfma_f32) {
      // dX = dY W^T + scaling (dY B^T) A^T: u = dY B^T (f32, [rows][rank]),
      // then the adapter term (A^T read through strides) on the kernel's MFMAs
      float* u = nullptr;
      int ld = (int)rank;
      if (lora) {
        u = at<float>(ws, L.dy_bt);
        if (adapter_row_product_supported(dy, lora->b, m, n, (int)rank)) {
          UNIFUR_HIP(launch_adapter_row_product(1, dy, false, lora->b, m, n, (int)rank, u, static_cast<unsigned*>(ws),
                                                kMaxCounters, stream));
          ld = adapter_row_product_ld((int)rank);
        } else {
          UNIFUR_HIP(launch_lora_xa_strided(dy, false, lora->b, 1, N, m, n, (int)rank, u, stream));
        }
      }
      F32GemmArgs a{};
      a.x = static_cast<const float*>(dy);
      a.packed = w->packed;
      a.scales = to_scales(w->scales);
      a.M = m;
      a.K = n;  // the reduction: d_out
      a.N = k;  // the outputs: d_in
      a.lora_xa = u;
      a.lora_ld = ld;
      a.lora_b = lora ? lora->a : nullptr;  // A^T: element (j, i) = A[i][j]
      a.lora_sbj = 1;
      a.lora_sbn = rank;
      a.lora_rank = (int)rank;
      a.lora_scaling = lora ? lora->scaling : 0.0f;
      a.y = dx;
      UNIFUR_HIP(launch_gemm_f32_mfma(a, w->scales.kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED, is_striped(w), true,
                                      dx_dtype == UNIFUR_NF4_BF16, stream));
    } else {
      const uint8_t* packed = nullptr;
      ScalesArg scales{};
      if (int r = row_major_view(w, ws, L.rm_codes, L.rm_scales, stream, &packed, &scales)) return r;
      float* wf = at<float>(ws, L.wf32);
      UNIFUR_HIP(launch_dequantize(packed, scales, (size_t)K * N, wf, false, u32_aligned(packed), stream));
      if (lora) UNIFUR_HIP(launch_lora_merge(wf, lora->a, lora->b, (int)rank, lora->scaling, K, N, wf, stream));
      Epilogue e{};
      e.y = dx;
      e.y_bf16 = dx_dtype == UNIFUR_NF4_BF16;
      // W' [K][N] row-major is the transposed [N_out = K][K_in = N] operand
      UNIFUR_HIP(launch_gemm_f32_wt(dy, dybf, wf, m, n, k, e, stream));
    }
  }
  if (mfma_grads) {
    if (!grads_done) UNIFUR_HIP(grads_on(stream));
  } else if (want_grads) {
    float* xa = at<float>(ws, L.xa);
    float* u = at<float>(ws, L.u);
    float* part = at<float>(ws, L.partials);
    const int r = (int)rank;
    if (grad_b) {
      // grad_B [r][N] = (x A)^T (dY scaling)
      UNIFUR_HIP(launch_narrow_mm(x, xbf, lora->a, false, m, k, r, part, xa, stream));
      UNIFUR_HIP(launch_narrow_atb(dy, dybf, xa, m, n, r, true, lora->scaling, part, grad_b, stream));
    }
    if (grad_a) {
      // grad_A [K][r] = x^T ((dY scaling) B^T)
      UNIFUR_HIP(launch_narrow_mm(dy, dybf, lora->b, true, m, n, r, part, u, stream));
      UNIFUR_HIP(launch_narrow_atb(x, xbf, u, m, k, r, false, lora->scaling, part, grad_a, stream));
    }
  }
  return UNIFUR_NF4_OK;
}


// ---------------------------------------------------- linears sharing x -----

// Up to three striped weights of one scale kind over the same x: one GEMV
// (<= 4 rows) or skinny (5..64 bf16 rows) launch covers them all, every
// activation load feeding every weight; otherwise the linears run in turn.
struct MultiLayout {
  bool fused, skinny;
  StripedPlan plan;
  size_t partials[kMaxGemvWeights];
  size_t total;  // fused plans; the sequential fallback sizes itself per linear
};

MultiLayout plan_multi(uint64_t rows, uint64_t d_in, const uint64_t* d_out, const unifur_nf4_weight* w, uint32_t n,
                       int x_dtype, const void* x) {
  MultiLayout L{};
  Carver c;
  bool ok = n >= 1 && n <= (uint32_t)kMaxGemvWeights && rows >= 1 && d_in <= 0x7fffffffu;
  for (uint32_t i = 0; ok && i < n; ++i)
    ok = d_out[i] % 64 == 0 && d_out[i] <= 0x7fffffffu && (!w || (is_striped(&w[i]) && w[i].d_in == d_in &&
                                                                    w[i].scales.kind == w[0].scales.kind));
  int dn[kMaxGemvWeights] = {};
  uint64_t stripes = 0;
  for (uint32_t i = 0; ok && i < n; ++i) {
    dn[i] = (int)d_out[i];
    stripes += d_out[i] / 16;
  }
  ok = ok && stripes / 4 <= (uint64_t)kMaxCounters;
  if (ok && rows <= (uint64_t)kGemvMaxRows) {
    L.fused = true;
    L.plan = plan_gemv_striped((int)rows, (int)d_in, dn, (int)n, false);
  } else if (ok && rows <= (uint64_t)kSkinnyMaxRows &&
             skinny_supported((int)rows, (int)d_in, x, x_dtype == UNIFUR_NF4_F32)) {
    L.fused = L.skinny = true;
    L.plan = plan_skinny((int)rows, (int)d_in, dn, (int)n, false);
    for (uint32_t i = 0; i < n; ++i)
      L.partials[i] = c.take(skinny_partial_floats(L.plan, (int)rows, dn[i]) * sizeof(float));
  }
  L.total = c.off;
  return L;
}

int run_linear_multi(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w, const float* const* bias,
                     void* const* y, int y_dtype, uint32_t n, void* workspace, uint64_t workspace_bytes,
                     hipStream_t stream) {
  UNIFUR_ARG(valid_dtype(x_dtype) && valid_dtype(y_dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  UNIFUR_ARG(n >= 1 && n <= (uint32_t)kMaxGemvWeights, "linear_forward_multi takes 1 to 3 weights");
  UNIFUR_ARG(w != nullptr && y != nullptr, "weights or outputs are NULL");
  for (uint32_t i = 0; i < n; ++i) {
    if (int r = check_weight(&w[i], "linear_forward_multi")) return r;
    UNIFUR_ARG(w[i].d_in == w[0].d_in, "the weights must share d_in");
    UNIFUR_ARG(rows == 0 || y[i] != nullptr, "an output is NULL");
  }
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x != nullptr, "x is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  for (uint32_t i = 0; i < n; ++i)
    UNIFUR_ARG(shape_fits(rows, w[i].d_in, w[i].d_out), "linear_forward_multi: shape too large (an element count over 2^48)");
  uint64_t d_out[kMaxGemvWeights] = {};
  for (uint32_t i = 0; i < n; ++i) d_out[i] = w[i].d_out;
  const MultiLayout L = plan_multi(rows, w[0].d_in, d_out, w, n, x_dtype, x);
  if (!L.fused) {
    for (uint32_t i = 0; i < n; ++i)
      if (int r = run_linear(x, x_dtype, rows, &w[i], bias ? bias[i] : nullptr, nullptr, y[i], y_dtype, workspace,
                             workspace_bytes, stream))
        return r;
    return UNIFUR_NF4_OK;
  }
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  GemvWeight gw[kMaxGemvWeights];
  for (uint32_t i = 0; i < n; ++i) {
    gw[i] = gemv_weight(&w[i], y[i], y_dtype == UNIFUR_NF4_BF16, at<unsigned>(ws, 0), at<float>(ws, L.partials[i]));
    gw[i].bias = bias ? bias[i] : nullptr;
  }
  if (L.skinny)
    UNIFUR_HIP(launch_skinny(L.plan, x, x_dtype == UNIFUR_NF4_F32, (int)rows, (int)w[0].d_in, gw, (int)n, false,
                             stream));
  else
    UNIFUR_HIP(launch_gemv_striped(L.plan, x, x_dtype == UNIFUR_NF4_BF16, (int)rows, (int)w[0].d_in, gw, (int)n,
                                   false, stream));
  return UNIFUR_NF4_OK;
}

// ------------------------------------------------ decoder-layer decode --
//
// The two halves of QwenDecoderLayer::step around the attention
// (src/qwennet.rs:1112-1129).  Workspace: the region a general-path call of
// run_linear / run_linear_multi / run_swiglu needs (it starts with the shared
// counter region), then this stage's own buffers.

size_t dtype_bytes(int dtype) { return dtype == UNIFUR_NF4_BF16 ? 2 : 4; }

int check_layer(const unifur_nf4_decoder_layer* l) {
  UNIFUR_ARG(l != nullptr, "decoder layer is NULL");
  if (int r = check_weight(&l->q, "q")) return r;
  if (int r = check_weight(&l->k, "k")) return r;
  if (int r = check_weight(&l->v, "v")) return r;
  if (int r = check_weight(&l->o, "o")) return r;
  if (int r = check_weight(&l->gate, "gate")) return r;
  if (int r = check_weight(&l->up, "up")) return r;
  if (int r = check_weight(&l->down, "down")) return r;
  const uint64_t h = l->q.d_in;
  UNIFUR_ARG(l->k.d_in == h && l->v.d_in == h, "q, k and v must share d_in (hidden)");
  UNIFUR_ARG(l->o.d_out == h, "o must map back to hidden");
  UNIFUR_ARG(l->gate.d_in == h && l->up.d_in == h && l->up.d_out == l->gate.d_out,
             "gate and up must be [hidden, intermediate]");
  UNIFUR_ARG(l->down.d_in == l->gate.d_out && l->down.d_out == h, "down must be [intermediate, hidden]");
  UNIFUR_ARG(l->input_norm != nullptr && l->post_norm != nullptr, "the norm weights are NULL");
  UNIFUR_ARG(h <= 0x7fffffffu && l->gate.d_out <= 0x7fffffffu, "dimension exceeds 2^31-1");
  return UNIFUR_NF4_OK;
}

// q, k, v in one striped GEMV launch with the input norm folded in
bool attn_in_fused(uint64_t rows, const unifur_nf4_decoder_layer* l) {
  const unifur_nf4_weight* w[3] = {&l->q, &l->k, &l->v};
  for (const auto* x : w)
    if (!is_striped(x) || x->scales.kind != l->q.scales.kind) return false;
  return rows >= 1 && rows <= (uint64_t)kGemvMaxRows;
}

// 5..64 bf16 (5..32 f32) rows: q, k, v in one skinny MFMA launch with the
// input norm folded in, when the three are striped with double-quantized
// scales, x suits the skinny kernel and its plan needs no d_in slabs
bool attn_in_skinny(uint64_t rows, const unifur_nf4_decoder_layer* l, const void* x, int dtype, StripedPlan* plan) {
  const unifur_nf4_weight* w[3] = {&l->q, &l->k, &l->v};
  for (const auto* t : w)
    if (!is_striped(t) || t->scales.kind != UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED) return false;
  const bool f32 = dtype == UNIFUR_NF4_F32;
  if (rows <= (uint64_t)kGemvMaxRows || !skinny_supported((int)rows, (int)l->q.d_in, x, f32)) return false;
  const int dn[3] = {(int)l->q.d_out, (int)l->k.d_out, (int)l->v.d_out};
  *plan = plan_skinny((int)rows, (int)l->q.d_in, dn, 3, false);
  return plan->splits == 1;
}

struct AttnInLayout {
  size_t inner, normed, total;
};

AttnInLayout plan_attn_in(uint64_t rows, const unifur_nf4_decoder_layer* l, int dtype) {
  AttnInLayout L{};
  const uint64_t dn[3] = {l->q.d_out, l->k.d_out, l->v.d_out};
  L.inner = align_up(std::max<uint64_t>(kCounterRegion,
                                        unifur_nf4_linear_multi_workspace_size(rows, l->q.d_in, dn, 3, dtype)));
  L.normed = L.inner;
  L.total = L.normed + align_up((size_t)rows * l->q.d_in * dtype_bytes(dtype));
  return L;
}

int run_attn_in(const void* x, int dtype, uint64_t rows, const unifur_nf4_decoder_layer* l, void* q, void* k,
                void* v, void* workspace, uint64_t workspace_bytes, hipStream_t stream) {
  UNIFUR_ARG(valid_dtype(dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (int r = check_layer(l)) return r;
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x != nullptr && q != nullptr && k != nullptr && v != nullptr, "x, q, k or v is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  UNIFUR_ARG(shape_fits(rows, l->q.d_in, l->gate.d_out), "decoder layer: shape too large (an element count over 2^48)");
  const bool bf = dtype == UNIFUR_NF4_BF16;
  const unifur_nf4_weight w[3] = {l->q, l->k, l->v};
  void* const outs[3] = {q, k, v};
  if (attn_in_fused(rows, l)) {
    int dn[3];
    GemvWeight gw[3];
    for (int i = 0; i < 3; ++i) {
      dn[i] = (int)w[i].d_out;
      gw[i] = gemv_weight(&w[i], outs[i], bf, nullptr, nullptr);
    }
    const StripedPlan plan = plan_gemv_striped((int)rows, (int)l->q.d_in, dn, 3, false);
    UNIFUR_HIP(launch_gemv_striped(plan, x, bf, (int)rows, (int)l->q.d_in, gw, 3, false, stream, l->input_norm,
                                   l->eps));
    return UNIFUR_NF4_OK;
  }
  StripedPlan sk{};
  if (attn_in_skinny(rows, l, x, dtype, &sk)) {
    GemvWeight gw[3];
    for (int i = 0; i < 3; ++i) gw[i] = gemv_weight(&w[i], outs[i], bf, nullptr, nullptr);
    UNIFUR_HIP(launch_skinny(sk, x, !bf, (int)rows, (int)l->q.d_in, gw, 3, false, stream, l->input_norm, l->eps));
    return UNIFUR_NF4_OK;
  }
  const AttnInLayout L = plan_attn_in(rows, l, dtype);
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  void* n = at<void>(ws, L.normed);
  UNIFUR_HIP(launch_rms_norm(x, bf, (int)rows, (int)l->q.d_in, l->input_norm, l->eps, n, bf, stream));
  return run_linear_multi(n, dtype, rows, w, nullptr, outs, dtype, 3, ws, L.inner, stream);
}

enum class OutPath { kGemv, kSkinny, kGeneral };
enum class MlpStage { kPairNorm, kMultiNorm, kSkinny, kGeneral };

struct AttnOutLayout {
  OutPath o_path;
  MlpStage mlp;
  StripedPlan o_plan, up_plan, down_plan;
  size_t inner, x1, nrm, tmp, h, u, hb, part0, part1, total;
};

AttnOutLayout plan_attn_out(uint64_t rows, const unifur_nf4_decoder_layer* l, int dtype, const void* ctx,
                            const void* x1_probe) {
  AttnOutLayout L{};
  const uint64_t hid = l->o.d_out, inter = l->gate.d_out, ctx_dim = l->o.d_in;
  const bool bf = dtype == UNIFUR_NF4_BF16;
  const int hd = (int)hid, gi[2] = {(int)inter, (int)inter};
  const bool mlp_striped = is_striped(&l->gate) && is_striped(&l->up) && is_striped(&l->down) &&
                           l->gate.scales.kind == l->up.scales.kind;
  // o with the residual in its epilogue
  if (is_striped(&l->o) && rows <= (uint64_t)kGemvMaxRows) {
    L.o_path = OutPath::kGemv;
    L.o_plan = plan_gemv_striped((int)rows, (int)ctx_dim, &hd, 1, false);
  } else if (is_striped(&l->o) && rows <= (uint64_t)kSkinnyMaxRows && ctx_dim <= 0x7fffffffu &&
             skinny_supported((int)rows, (int)ctx_dim, ctx, !bf) && hid / 64 <= (uint64_t)kMaxCounters) {
    L.o_path = OutPath::kSkinny;
    L.o_plan = plan_skinny((int)rows, (int)ctx_dim, &hd, 1, false);
  } else {
    L.o_path = OutPath::kGeneral;
  }
  // gate/up (+ norm) then down with the residual in its epilogue
  if (mlp_striped && rows <= (uint64_t)kGemvPairMaxRows) {
    L.mlp = MlpStage::kPairNorm;
    L.up_plan = plan_gemv_striped((int)rows, (int)hid, gi, 2, true);
    L.down_plan = plan_gemv_striped((int)rows, (int)inter, &hd, 1, false);
  } else if (mlp_striped && rows <= (uint64_t)kGemvMaxRows) {
    L.mlp = MlpStage::kMultiNorm;
    L.up_plan = plan_gemv_striped((int)rows, (int)hid, gi, 2, false);
    L.down_plan = plan_gemv_striped((int)rows, (int)inter, &hd, 1, false);
  } else if (mlp_striped && rows <= (uint64_t)kSkinnyMaxRows && skinny_supported((int)rows, (int)hid, x1_probe, !bf) &&
             skinny_supported((int)rows, (int)inter, x1_probe, !bf) &&
             std::max(hid, inter) / 64 <= (uint64_t)kMaxCounters) {
    L.mlp = MlpStage::kSkinny;
    L.up_plan = plan_skinny((int)rows, (int)hid, gi, 2, true);
    L.down_plan = plan_skinny((int)rows, (int)inter, &hd, 1, false);
  } else {
    L.mlp = MlpStage::kGeneral;
  }
  uint64_t inner = kCounterRegion;
  if (L.o_path == OutPath::kGeneral) {
    // the o linear's own plan for this ctx (a misaligned ctx can take the
    // generic path, which needs more than the aligned size query says)
    inner = std::max<uint64_t>(inner, unifur_nf4_linear_workspace_size(rows, ctx_dim, hid, dtype, 0));
    inner = std::max<uint64_t>(inner, plan_linear(rows, ctx_dim, hid, 0, l->o.packed, dtype, ctx, is_striped(&l->o),
                                                  l->o.scales.kind).total);
  }
  if (L.mlp == MlpStage::kGeneral)
    inner = std::max<uint64_t>(inner, swiglu_workspace(rows, hid, inter, dtype, true));
  Carver c;
  c.off = align_up(inner);
  L.inner = c.off;
  const size_t act = (size_t)rows * hid * dtype_bytes(dtype);
  L.x1 = c.take(act);
  L.nrm = c.take(act);
  L.tmp = c.take(act);
  L.h = c.take((size_t)rows * inter * 4);
  L.u = c.take((size_t)rows * inter * 4);
  L.hb = c.take((size_t)rows * inter * 2);
  size_t p0 = 0, p1 = 0;
  if (L.o_path == OutPath::kSkinny) p0 = skinny_partial_floats(L.o_plan, (int)rows, hd);
  if (L.mlp == MlpStage::kSkinny) {
    p0 = std::max(p0, std::max(skinny_partial_floats(L.up_plan, (int)rows, (int)inter),
                               skinny_partial_floats(L.down_plan, (int)rows, hd)));
    p1 = skinny_partial_floats(L.up_plan, (int)rows, (int)inter);
  }
  L.part0 = c.take(p0 * sizeof(float));
  L.part1 = c.take(p1 * sizeof(float));
  L.total = c.off;
  return L;
}

int run_attn_out_mlp(const void* x, const void* ctx, int dtype, uint64_t rows, const unifur_nf4_decoder_layer* l,
                     void* y, void* workspace, uint64_t workspace_bytes, hipStream_t stream) {
  UNIFUR_ARG(valid_dtype(dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (int r = check_layer(l)) return r;
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x != nullptr && ctx != nullptr && y != nullptr, "x, ctx or y is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  UNIFUR_ARG(shape_fits(rows, l->q.d_in, l->gate.d_out), "decoder layer: shape too large (an element count over 2^48)");
  const bool bf = dtype == UNIFUR_NF4_BF16;
  const uint64_t hid = l->o.d_out, inter = l->gate.d_out;
  const AttnOutLayout L = plan_attn_out(rows, l, dtype, ctx, reinterpret_cast<const void*>(uintptr_t{256}));
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  unsigned* cnt = at<unsigned>(ws, 0);
  void* x1 = at<void>(ws, L.x1);
  // x1 = x + ctx Wo
  if (L.o_path == OutPath::kGeneral) {
    void* t = at<void>(ws, L.tmp);
    if (int r = run_linear(ctx, dtype, rows, &l->o, nullptr, nullptr, t, dtype, ws, L.inner, stream)) return r;
    UNIFUR_HIP(launch_add(x, t, bf, (size_t)rows * hid, x1, stream));
  } else {
    GemvWeight ow = gemv_weight(&l->o, x1, bf, cnt, at<float>(ws, L.part0));
    ow.residual = x;
    if (L.o_path == OutPath::kGemv)
      UNIFUR_HIP(launch_gemv_striped(L.o_plan, ctx, bf, (int)rows, (int)l->o.d_in, &ow, 1, false, stream));
    else
      UNIFUR_HIP(launch_skinny(L.o_plan, ctx, !bf, (int)rows, (int)l->o.d_in, &ow, 1, false, stream));
  }
  // y = x1 + down(silu(gate n) * up n), n = post_norm(x1)
  float* h = at<float>(ws, L.h);
  switch (L.mlp) {
    case MlpStage::kPairNorm:
    case MlpStage::kMultiNorm: {
      const bool pair = L.mlp == MlpStage::kPairNorm;
      GemvWeight gw[2] = {gemv_weight(&l->gate, h, false, cnt, nullptr),
                          gemv_weight(&l->up, pair ? nullptr : at<float>(ws, L.u), false, cnt, nullptr)};
      UNIFUR_HIP(launch_gemv_striped(L.up_plan, x1, bf, (int)rows, (int)hid, gw, 2, pair, stream, l->post_norm,
                                     l->eps));
      if (!pair) UNIFUR_HIP(launch_silu_mul(h, at<float>(ws, L.u), (size_t)rows * inter, h, stream));
      GemvWeight dw = gemv_weight(&l->down, y, bf, cnt, nullptr);
      dw.residual = x1;
      UNIFUR_HIP(launch_gemv_striped(L.down_plan, h, false, (int)rows, (int)inter, &dw, 1, false, stream));
      return UNIFUR_NF4_OK;
    }
    case MlpStage::kSkinny: {
      // the SwiGLU middle in the stage's dtype; the post norm folded into the
      // gate/up launch (double-quantized scales, no d_in slabs), else n =
      // post_norm(x1) first
      void* mid = bf ? at<void>(ws, L.hb) : static_cast<void*>(h);
      float* p0 = at<float>(ws, L.part0);
      GemvWeight gw[2] = {gemv_weight(&l->gate, mid, bf, cnt, p0),
                          gemv_weight(&l->up, nullptr, bf, cnt, at<float>(ws, L.part1))};
      if (l->gate.scales.kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED && L.up_plan.splits == 1) {
        UNIFUR_HIP(launch_skinny(L.up_plan, x1, !bf, (int)rows, (int)hid, gw, 2, true, stream, l->post_norm, l->eps));
      } else {
        void* n = at<void>(ws, L.nrm);
        UNIFUR_HIP(launch_rms_norm(x1, bf, (int)rows, (int)hid, l->post_norm, l->eps, n, bf, stream));
        UNIFUR_HIP(launch_skinny(L.up_plan, n, !bf, (int)rows, (int)hid, gw, 2, true, stream));
      }
      GemvWeight dw = gemv_weight(&l->down, y, bf, cnt, p0);
      dw.residual = x1;
      UNIFUR_HIP(launch_skinny(L.down_plan, mid, !bf, (int)rows, (int)inter, &dw, 1, false, stream));
      return UNIFUR_NF4_OK;
    }
    case MlpStage::kGeneral:
      break;
  }
  void* n = at<void>(ws, L.nrm);
  void* t = at<void>(ws, L.tmp);
  UNIFUR_HIP(launch_rms_norm(x1, bf, (int)rows, (int)hid, l->post_norm, l->eps, n, bf, stream));
  if (int r = run_swiglu(n, dtype, rows, &l->gate, &l->up, &l->down, t, dtype, ws, L.inner, stream)) return r;
  UNIFUR_HIP(launch_add(x1, t, bf, (size_t)rows * hid, y, stream));
  return UNIFUR_NF4_OK;
}

// ------------------------------------------------- allocation-free entry --

// The scratch of unifur_nf4_linear_forward_noalloc: a file-scope device array,
// one copy per GPU the library runs on, held until the process ends.  In host
// code its name is only a symbol: kernels and fills get the per-device address
// that hipGetSymbolAddress returns, kept in static_scratch().
constexpr size_t kStaticScratchBytes = size_t{16} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

__global__ void zero_words_kernel(uint32_t* p, size_t words) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

struct StaticScratch {
  std::mutex mu;
  std::map<int, void*> ptr;  // device -> address of its copy of `scratch`
  // Ordering of the calls that share a device's scratch: the event recorded
  // after the last eager call's launches and that call's stream.
  std::mutex order_mu;
  std::map<int, hipEvent_t> done;
  std::map<int, hipStream_t> last;
};

StaticScratch& static_scratch() {
  static StaticScratch* s = new StaticScratch();  // never destroyed, like the workspaces
  return *s;
}

// Set-up on the first call on a device, with that device current: look up
// this device's address of `scratch` and clear its arrival-counter region
// (the only part a call expects to find zero; every call leaves it zero) with
// a fill kernel on the caller's stream, ahead of the call's own launches.  A
// first call under stream capture records that fill in the graph and sets up
// again on the next call.
int static_scratch_address(hipStream_t stream, void** out) {
  int dev = 0;
  UNIFUR_HIP(hipGetDevice(&dev));
  StaticScratch& s = static_scratch();
  std::lock_guard<std::mutex> lock(s.mu);
  const auto it = s.ptr.find(dev);
  if (it != s.ptr.end()) {
    *out = it->second;
    return UNIFUR_NF4_OK;
  }
  void* p = nullptr;
  UNIFUR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  if (p == nullptr) return fail(UNIFUR_NF4_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch");
  zero_words_kernel<<<16, 256, 0, stream>>>(static_cast<uint32_t*>(p), kCounterRegion / sizeof(uint32_t));
  UNIFUR_HIP(hipGetLastError());
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  UNIFUR_HIP(hipStreamIsCapturing(stream, &cap));
  if (cap == hipStreamCaptureStatusNone) s.ptr[dev] = p;
  *out = p;
  return UNIFUR_NF4_OK;
}

int run_linear_noalloc(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w, const float* bias,
                       const unifur_nf4_lora* lora, void* y, int y_dtype, hipStream_t stream) {
  UNIFUR_ARG(valid_dtype(x_dtype) && valid_dtype(y_dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (int r = check_weight(w, "linear")) return r;
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x != nullptr && y != nullptr, "x or y is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  UNIFUR_ARG(shape_fits(rows, w->d_in, w->d_out), "linear: shape too large (an element count over 2^48)");
  const uint32_t rank = lora ? lora->rank : 0;
  if (lora) UNIFUR_ARG(rank >= 1 && rank <= 64, "lora rank must be in [1, 64]");
  LinearLayout L =
      plan_linear(rows, w->d_in, w->d_out, rank, w->packed, x_dtype, x, is_striped(w), w->scales.kind, false);
  if (L.total > kStaticScratchBytes)  // without the split-K partials
    L = plan_linear(rows, w->d_in, w->d_out, rank, w->packed, x_dtype, x, is_striped(w), w->scales.kind, false, false);
  if (L.total > kStaticScratchBytes)
    return fail(UNIFUR_NF4_ERR_WORKSPACE, "linear_forward_noalloc: this call needs " + std::to_string(L.total) +
                                              " bytes of scratch, the allocation-free entry point holds " +
                                              std::to_string(kStaticScratchBytes));
  // Calls on one GPU share its scratch.  An eager call on another stream
  // than the previous eager call's first waits on the GPU for that call's
  // work (an event recorded after its launches, the set-up's fill included),
  // and the lock keeps a second host thread from launching in between, so
  // calls from different streams and threads run one after the other
  // instead of racing.  Calls made under stream capture are not ordered this
  // way (their replays are the caller's to order).
  StaticScratch& s = static_scratch();
  std::lock_guard<std::mutex> lock(s.order_mu);
  void* p = nullptr;
  if (int r = static_scratch_address(stream, &p)) return r;
  int dev = 0;
  UNIFUR_HIP(hipGetDevice(&dev));
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  UNIFUR_HIP(hipStreamIsCapturing(stream, &cap));
  const bool eager = cap == hipStreamCaptureStatusNone;
  hipEvent_t* ev = nullptr;
  if (eager) {
    ev = &s.done[dev];
    if (*ev == nullptr) UNIFUR_HIP(hipEventCreateWithFlags(ev, hipEventDisableTiming));  // set-up, once per device
    const auto it = s.last.find(dev);
    if (it != s.last.end() && it->second != stream) UNIFUR_HIP(hipStreamWaitEvent(stream, *ev, 0));
  }
  const int r = run_linear(x, x_dtype, rows, w, bias, lora, y, y_dtype, p, kStaticScratchBytes, stream, false);
  if (eager) {
    UNIFUR_HIP(hipEventRecord(*ev, stream));
    s.last[dev] = stream;
  }
  return r;
}

}  // namespace
}  // namespace unifur

using namespace unifur;

extern "C" {

const char* unifur_nf4_last_error(void) { return g_last_error.c_str(); }

int unifur_nf4_levels(float out[16]) {
  UNIFUR_ARG(out != nullptr, "out is NULL");
  for (int c = 0; c < 16; ++c) {
    const uint32_t b = level_bits(c);
    std::memcpy(&out[c], &b, 4);
  }
  return UNIFUR_NF4_OK;
}

uint64_t unifur_nf4_num_blocks(uint64_t len) { return ceil_div_u64(len, UNIFUR_NF4_BLOCK_SIZE); }

uint64_t unifur_nf4_packed_bytes(uint64_t len) { return ceil_div_u64(len, 2); }

uint64_t unifur_nf4_estimated_resident_bytes(uint64_t len, int double_quantized) {
  const uint64_t blocks = unifur_nf4_num_blocks(len);
  return unifur_nf4_packed_bytes(len) + (double_quantized ? blocks + 4 : 4 * blocks);
}

double unifur_nf4_bits_per_value(uint64_t len, int double_quantized) {
  if (len == 0) return 0.0;
  return 8.0 * (double)unifur_nf4_estimated_resident_bytes(len, double_quantized) / (double)len;
}

double unifur_nf4_simulated_bits_per_value(uint64_t len, int double_quantized) {
  if (len == 0) return 0.0;
  const double blocks = (double)unifur_nf4_num_blocks(len);
  const double payload = 4.0 * (double)len;
  const double scales = double_quantized ? 8.0 * blocks + 32.0 : 32.0 * blocks;
  return (payload + scales) / (double)len;
}

int unifur_nf4_quantize(const float* values, uint64_t len, uint8_t* packed, float* absmax, void* stream) {
  if (len == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(values && packed && absmax, "values, packed or absmax is NULL");
  const bool aligned = (reinterpret_cast<uintptr_t>(values) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(packed) & 1u) == 0;
  UNIFUR_HIP(launch_quantize(values, len, packed, absmax, aligned, static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_double_quantize(const float* absmax, uint64_t num_blocks, uint8_t* dq_codes, float* scale_of_scales,
                               void* stream) {
  UNIFUR_ARG(scale_of_scales != nullptr, "scale_of_scales is NULL");
  UNIFUR_ARG(num_blocks == 0 || (absmax && dq_codes), "absmax or dq_codes is NULL");
  UNIFUR_HIP(launch_double_quantize(absmax, num_blocks, dq_codes, scale_of_scales, static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_dequantize(const uint8_t* packed, const unifur_nf4_scales* scales, uint64_t len, void* out,
                          int out_dtype, void* stream) {
  UNIFUR_ARG(valid_dtype(out_dtype), "out_dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (len == 0) return UNIFUR_NF4_OK;  // an empty tensor holds no scales to validate
  if (int r = check_scales(scales)) return r;
  UNIFUR_ARG(packed && out, "packed or out is NULL");
  const bool aligned = (reinterpret_cast<uintptr_t>(packed) & 3u) == 0 &&
                       (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  UNIFUR_HIP(launch_dequantize(packed, to_scales(*scales), len, out, out_dtype == UNIFUR_NF4_BF16, aligned,
                               static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_unpack_codes(const uint8_t* packed, uint64_t len, uint8_t* codes, void* stream) {
  if (len == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(packed && codes, "packed or codes is NULL");
  UNIFUR_HIP(launch_unpack_codes(packed, len, codes, static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_pack_codes(const uint8_t* codes, uint64_t len, uint8_t* packed, void* stream) {
  if (len == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(packed && codes, "packed or codes is NULL");
  UNIFUR_HIP(launch_pack_codes(codes, len, packed, static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

uint64_t unifur_nf4_decoder_attn_in_workspace_size(uint64_t rows, const unifur_nf4_decoder_layer* layer, int dtype) {
  if (rows == 0 || check_layer(layer) != UNIFUR_NF4_OK || !valid_dtype(dtype)) return 0;
  if (rows > 0x7fffffffu || !shape_fits(rows, layer->q.d_in, layer->gate.d_out)) return UINT64_MAX;
  if (attn_in_fused(rows, layer)) return 0;
  return plan_attn_in(rows, layer, dtype).total;
}

int unifur_nf4_decoder_attn_in(const void* x, int dtype, uint64_t rows, const unifur_nf4_decoder_layer* layer,
                               void* q, void* k, void* v, void* workspace, uint64_t workspace_bytes, void* stream) {
  return run_attn_in(x, dtype, rows, layer, q, k, v, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

uint64_t unifur_nf4_decoder_attn_out_mlp_workspace_size(uint64_t rows, const unifur_nf4_decoder_layer* layer,
                                                        int dtype) {
  if (rows == 0 || check_layer(layer) != UNIFUR_NF4_OK || !valid_dtype(dtype)) return 0;
  if (rows > 0x7fffffffu || !shape_fits(rows, layer->q.d_in, layer->gate.d_out)) return UINT64_MAX;
  // a ctx off the 16-byte alignment can move the o projection to the
  // general path, whose workspace differs: the larger of both plans
  const void* aligned = reinterpret_cast<const void*>(uintptr_t{256});
  const void* ragged = reinterpret_cast<const void*>(uintptr_t{256} + (dtype == UNIFUR_NF4_BF16 ? 2 : 4));
  return std::max<uint64_t>(plan_attn_out(rows, layer, dtype, aligned, aligned).total,
                            plan_attn_out(rows, layer, dtype, ragged, aligned).total);
}

int unifur_nf4_decoder_attn_out_mlp(const void* x, const void* ctx, int dtype, uint64_t rows,
                                    const unifur_nf4_decoder_layer* layer, void* y, void* workspace,
                                    uint64_t workspace_bytes, void* stream) {
  return run_attn_out_mlp(x, ctx, dtype, rows, layer, y, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

uint64_t unifur_nf4_linear_multi_workspace_size(uint64_t rows, uint64_t d_in, const uint64_t* d_out, uint32_t n,
                                                int x_dtype) {
  if (rows == 0 || d_in == 0 || !d_out || n == 0 || n > (uint32_t)kMaxGemvWeights) return 0;
  for (uint32_t i = 0; i < n; ++i)
    if (rows > 0x7fffffffu || !shape_fits(rows, d_in, d_out[i])) return UINT64_MAX;
  const void* aligned = reinterpret_cast<const void*>(uintptr_t{256});
  const MultiLayout L = plan_multi(rows, d_in, d_out, nullptr, n, x_dtype, aligned);
  uint64_t need = L.total;
  for (uint32_t i = 0; i < n; ++i)  // the linears one at a time, when not fused
    need = std::max<uint64_t>(need, unifur_nf4_linear_workspace_size(rows, d_in, d_out[i], x_dtype, 0));
  return need;
}

int unifur_nf4_linear_forward_multi(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w,
                                    const float* const* bias, void* const* y, int y_dtype, uint32_t n,
                                    void* workspace, uint64_t workspace_bytes, void* stream) {
  return run_linear_multi(x, x_dtype, rows, w, bias, y, y_dtype, n, workspace, workspace_bytes,
                          static_cast<hipStream_t>(stream));
}

uint64_t unifur_nf4_linear_backward_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int dy_dtype,
                                                   uint32_t lora_rank) {
  if (d_in == 0 || d_out == 0) return 0;
  if (rows > 0x7fffffffu || !shape_fits(rows, d_in, d_out)) return UINT64_MAX;
  uint64_t need = 0;
  for (int striped = 0; striped < 2; ++striped)
    for (int kind = 0; kind < 2; ++kind)
      need = std::max<uint64_t>(need, plan_backward(rows, d_in, d_out, lora_rank, dy_dtype, rows > 0, lora_rank > 0,
                                                    striped && d_out % 64 == 0, kind, true)
                                          .total);
  return need;
}

uint64_t unifur_nf4_linear_backward_min_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int dy_dtype,
                                                       uint32_t lora_rank, int layout) {
  if (d_in == 0 || d_out == 0) return 0;
  if (rows > 0x7fffffffu || !shape_fits(rows, d_in, d_out)) return UINT64_MAX;
  // only a striped weight can take the fused dX kernel; any other layout
  // (or an unknown value) gets the default size
  if (layout != UNIFUR_NF4_LAYOUT_STRIPED || d_out % 64 != 0)
    return unifur_nf4_linear_backward_workspace_size(rows, d_in, d_out, dy_dtype, lora_rank);
  uint64_t need = 0;
  for (int kind = 0; kind < 2; ++kind) {
    const BackwardLayout L = plan_backward(rows, d_in, d_out, lora_rank, dy_dtype, rows > 0, lora_rank > 0,
                                           true, kind, true, false, false);
    if (rows > 0 && !L.fused) return unifur_nf4_linear_backward_workspace_size(rows, d_in, d_out, dy_dtype, lora_rank);
    need = std::max<uint64_t>(need, L.total);
  }
  return need;
}

int unifur_nf4_linear_backward(const void* dy, int dy_dtype, uint64_t rows, const unifur_nf4_weight* w,
                               const unifur_nf4_lora* lora, const void* x, int x_dtype, void* dx, int dx_dtype,
                               float* grad_a, float* grad_b, void* workspace, uint64_t workspace_bytes,
                               void* stream) {
  return run_backward(dy, dy_dtype, rows, w, lora, x, x_dtype, dx, dx_dtype, grad_a, grad_b, workspace,
                      workspace_bytes, static_cast<hipStream_t>(stream));
}

int unifur_nf4_embedding_forward(const uint8_t* packed, const unifur_nf4_scales* scales, uint64_t n_embedding,
                                 uint64_t d_model, const void* ids, int ids_dtype, uint64_t n_ids, void* out,
                                 int out_dtype, void* stream) {
  UNIFUR_ARG(valid_dtype(out_dtype), "out_dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  UNIFUR_ARG(ids_dtype == UNIFUR_NF4_IDS_I32 || ids_dtype == UNIFUR_NF4_IDS_I64,
             "ids_dtype must be UNIFUR_NF4_IDS_I32 or UNIFUR_NF4_IDS_I64");
  if (n_ids == 0 || d_model == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(ids && out, "ids or out is NULL");
  UNIFUR_ARG(fits_elements(n_ids, d_model) && fits_elements(n_embedding, d_model),
             "embedding: shape too large (an element count over 2^48)");
  if (n_embedding > 0) {
    if (int r = check_scales(scales)) return r;
    UNIFUR_ARG(packed != nullptr, "packed is NULL");
  }
  UNIFUR_ARG(aligned_to(ids, ids_dtype == UNIFUR_NF4_IDS_I64 ? 8 : 4), "ids misaligned for its type");
  UNIFUR_ARG(aligned_to(out, out_dtype == UNIFUR_NF4_BF16 ? 2 : 4), "out misaligned for its dtype");
  const ScalesArg sc = n_embedding > 0 ? to_scales(*scales) : ScalesArg{};
  UNIFUR_HIP(launch_embedding(packed, sc, n_embedding, d_model, ids, ids_dtype == UNIFUR_NF4_IDS_I64, n_ids, out,
                              out_dtype == UNIFUR_NF4_BF16, static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

uint64_t unifur_nf4_linear_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int x_dtype,
                                          uint32_t lora_rank) {
  if (rows == 0 || d_in == 0 || d_out == 0) return 0;
  if (rows > 0x7fffffffu || !shape_fits(rows, d_in, d_out)) return UINT64_MAX;
  // sized for 16-byte-aligned buffers, as hipMalloc returns them; a call
  // with misaligned buffers may take the generic path, which needs more and
  // reports UNIFUR_NF4_ERR_WORKSPACE with the size when given less
  const void* aligned = reinterpret_cast<const void*>(uintptr_t{256});
  uint64_t need = 0;
  for (int striped = 0; striped < 2; ++striped)
    for (int kind = 0; kind < 2; ++kind)
      need = std::max<uint64_t>(need, plan_linear(rows, d_in, d_out, lora_rank, aligned, x_dtype, aligned,
                                                  striped && d_out % 64 == 0, kind).total);
  return need;
}

uint64_t unifur_nf4_linear_min_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int x_dtype,
                                              uint32_t lora_rank) {
  if (rows == 0 || d_in == 0 || d_out == 0) return 0;
  if (rows > 0x7fffffffu || !shape_fits(rows, d_in, d_out)) return UINT64_MAX;
  const void* aligned = reinterpret_cast<const void*>(uintptr_t{256});
  uint64_t need = 0;
  for (int striped = 0; striped < 2; ++striped)
    for (int kind = 0; kind < 2; ++kind)
      need = std::max<uint64_t>(need, plan_linear(rows, d_in, d_out, lora_rank, aligned, x_dtype, aligned,
                                                  striped && d_out % 64 == 0, kind, false, false).total);
  return need;
}

uint64_t unifur_nf4_swiglu_min_workspace_size(uint64_t rows, uint64_t hidden, uint64_t intermediate, int x_dtype) {
  return swiglu_workspace(rows, hidden, intermediate, x_dtype, false, false);
}

int unifur_nf4_linear_forward(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w,
                              const float* bias, const unifur_nf4_lora* lora, void* y, int y_dtype, void* workspace,
                              uint64_t workspace_bytes, void* stream) {
  return run_linear(x, x_dtype, rows, w, bias, lora, y, y_dtype, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

int unifur_nf4_linear_forward_noalloc(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w,
                                      const float* bias, const unifur_nf4_lora* lora, void* y, int y_dtype,
                                      void* stream) {
  return run_linear_noalloc(x, x_dtype, rows, w, bias, lora, y, y_dtype, static_cast<hipStream_t>(stream));
}

int unifur_nf4_qlora_forward(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w,
                             const unifur_nf4_lora* lora, void* y, int y_dtype, void* workspace,
                             uint64_t workspace_bytes, void* stream) {
  UNIFUR_ARG(lora != nullptr, "qlora_forward needs a lora adapter");
  return run_linear(x, x_dtype, rows, w, nullptr, lora, y, y_dtype, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

uint64_t unifur_nf4_swiglu_workspace_size(uint64_t rows, uint64_t hidden, uint64_t intermediate, int x_dtype) {
  return swiglu_workspace(rows, hidden, intermediate, x_dtype, true);
}
int unifur_nf4_quantize_transposed(const void* src, int src_dtype, uint64_t out_features, uint64_t in_features,
                                   uint8_t* packed, float* absmax, void* stream) {
  UNIFUR_ARG(valid_src_dtype(src_dtype), "src_dtype must be UNIFUR_NF4_F32, UNIFUR_NF4_BF16 or UNIFUR_NF4_F16");
  if (out_features == 0 || in_features == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(src && packed && absmax, "src, packed or absmax is NULL");
  UNIFUR_ARG(out_features % 64 == 0, "quantize_transposed needs out_features % 64 == 0");
  UNIFUR_ARG(out_features / 64 <= 65535u && in_features <= 0x7fffffffffull, "quantize_transposed: shape too large");
  UNIFUR_ARG(aligned_to(packed, 8), "packed must be 8-byte aligned");
  UNIFUR_ARG(aligned_to(src, src_dtype == UNIFUR_NF4_F32 ? 4 : 2), "src is misaligned for its dtype");
  UNIFUR_HIP(launch_quantize_transposed(src, src_kind_of(src_dtype), out_features, in_features, packed, absmax,
                                        static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

uint64_t unifur_nf4_quantize_linears_workspace_size(const uint64_t* d_in, const uint64_t* d_out, uint32_t n) {
  if (n == 0 || !d_in || !d_out) return 0;
  for (uint32_t i = 0; i < n; ++i)
    if (!fits_elements(d_in[i], d_out[i])) return UINT64_MAX;
  Carver c;
  c.take(quantize_linears_scratch_bytes(d_in, d_out, n));
  return c.off;
}

namespace {

int run_quantize_linears(const void* const* values, int src_kind, const uint64_t* d_in, const uint64_t* d_out,
                         uint32_t n, uint8_t* const* packed, uint8_t* const* dq_codes,
                         float* const* scale_of_scales, void* workspace, uint64_t workspace_bytes, void* stream) {
  if (n == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(values && d_in && d_out && packed && dq_codes && scale_of_scales, "an argument array is NULL");
  const uintptr_t align = src_kind == kQuantSrcF32 ? 16 : src_kind == kQuantSrcF32T ? 4 : 2;
  for (uint32_t i = 0; i < n; ++i) {
    UNIFUR_ARG(d_in[i] > 0 && d_out[i] > 0 && d_out[i] % 64 == 0, "quantize_linears needs d_out % 64 == 0");
    UNIFUR_ARG(d_in[i] <= 0x7fffffffu && d_out[i] <= 0x7fffffffu && fits_elements(d_in[i], d_out[i]),
               "quantize_linears: weight too large");
    UNIFUR_ARG(values[i] && packed[i] && dq_codes[i] && scale_of_scales[i], "a tensor pointer is NULL");
    UNIFUR_ARG(aligned_to(values[i], align) && aligned_to(packed[i], 8) && aligned_to(scale_of_scales[i], 4),
               src_kind == kQuantSrcF32 ? "values must be 16-byte, packed 8-byte aligned"
                                        : "values must be aligned to their dtype, packed 8-byte aligned");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t need = quantize_linears_scratch_bytes(d_in, d_out, n);
  void* ws = nullptr;
  Carver c;
  const size_t off = c.take(need);
  if (int r = resolve_workspace(workspace, workspace_bytes, c.off, st, &ws)) return r;
  UNIFUR_HIP(launch_quantize_linears(values, src_kind, d_in, d_out, n, packed, dq_codes, scale_of_scales,
                                     at<void>(ws, off), st));
  return UNIFUR_NF4_OK;
}

}  // namespace

int unifur_nf4_quantize_linears(const float* const* values, const uint64_t* d_in, const uint64_t* d_out, uint32_t n,
                                uint8_t* const* packed, uint8_t* const* dq_codes, float* const* scale_of_scales,
                                void* workspace, uint64_t workspace_bytes, void* stream) {
  return run_quantize_linears(reinterpret_cast<const void* const*>(values), kQuantSrcF32, d_in, d_out, n, packed,
                              dq_codes, scale_of_scales, workspace, workspace_bytes, stream);
}

int unifur_nf4_transpose_checkpoint(const void* src, int src_dtype, uint64_t out_features, uint64_t in_features,
                                    float* dst, void* stream) {
  UNIFUR_ARG(valid_src_dtype(src_dtype), "src_dtype must be UNIFUR_NF4_F32, UNIFUR_NF4_BF16 or UNIFUR_NF4_F16");
  if (out_features == 0 || in_features == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(src && dst, "src or dst is NULL");
  UNIFUR_ARG(out_features <= 65535ull * 64ull, "out_features exceeds 65535 * 64");
  UNIFUR_ARG(aligned_to(src, src_dtype == UNIFUR_NF4_F32 ? 4 : 2) && aligned_to(dst, 4),
             "src or dst misaligned for its dtype");
  UNIFUR_HIP(launch_transpose_decode(src, src_kind_of(src_dtype), out_features, in_features, dst,
                                     static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_quantize_checkpoint_linears(const void* const* values, int src_dtype, const uint64_t* d_in,
                                           const uint64_t* d_out, uint32_t n, uint8_t* const* packed,
                                           uint8_t* const* dq_codes, float* const* scale_of_scales, void* workspace,
                                           uint64_t workspace_bytes, void* stream) {
  UNIFUR_ARG(valid_src_dtype(src_dtype), "src_dtype must be UNIFUR_NF4_F32, UNIFUR_NF4_BF16 or UNIFUR_NF4_F16");
  const int kind = src_dtype == UNIFUR_NF4_BF16 ? kQuantSrcBf16T : src_dtype == UNIFUR_NF4_F16 ? kQuantSrcF16T
                                                                                              : kQuantSrcF32T;
  return run_quantize_linears(values, kind, d_in, d_out, n, packed, dq_codes, scale_of_scales, workspace,
                              workspace_bytes, stream);
}

uint64_t unifur_nf4_dense_linear_workspace_size(uint64_t rows, uint32_t lora_rank) {
  if (rows == 0 || lora_rank == 0) return 0;
  if (!fits_elements(rows, lora_rank)) return UINT64_MAX;
  Carver c;
  c.take((size_t)rows * lora_rank * sizeof(float));
  return c.off;
}

int unifur_nf4_dense_linear_forward(const void* x, int x_dtype, uint64_t rows, const float* w, uint64_t d_in,
                                    uint64_t d_out, const float* bias, const unifur_nf4_lora* lora, void* y,
                                    int y_dtype, void* workspace, uint64_t workspace_bytes, void* stream) {
  UNIFUR_ARG(valid_dtype(x_dtype) && valid_dtype(y_dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  UNIFUR_ARG(d_in > 0 && d_out > 0 && d_in <= 0x7fffffffu && d_out <= 0x7fffffffu, "bad weight shape");
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x && y && w, "x, y or w is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  const uint32_t rank = lora ? lora->rank : 0;
  if (lora) {
    UNIFUR_ARG(lora->a != nullptr && lora->b != nullptr, "lora factors are NULL");
    UNIFUR_ARG(rank >= 1 && rank <= 64, "lora rank must be in [1, 64]");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t need = lora ? (size_t)rows * rank * sizeof(float) : 0;
  void* ws = nullptr;
  if (need) {
    // the counter region keeps its offset-0 meaning for shared workspaces
    Carver c;
    const size_t off = c.take(need);
    if (int r = resolve_workspace(workspace, workspace_bytes, c.off, st, &ws)) return r;
    ws = at<char>(ws, off);
  }
  float* xa = static_cast<float*>(ws);
  if (lora) UNIFUR_HIP(launch_lora_xa(x, x_dtype == UNIFUR_NF4_BF16, lora->a, (int)rows, (int)d_in, (int)rank, xa, st));
  Epilogue e{bias, xa, lora ? lora->b : nullptr, (int)rank, lora ? lora->scaling : 0.0f, y,
             y_dtype == UNIFUR_NF4_BF16};
  UNIFUR_HIP(launch_gemm_f32(x, x_dtype == UNIFUR_NF4_BF16, w, (int)rows, (int)d_in, (int)d_out, e, st));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_lora_merge(const float* w, uint64_t d_in, uint64_t d_out, const unifur_nf4_lora* lora, float* out,
                          void* stream) {
  UNIFUR_ARG(lora != nullptr && lora->a && lora->b, "lora factors are NULL");
  UNIFUR_ARG(lora->rank >= 1, "lora rank must be positive");
  if (d_in == 0 || d_out == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(w && out, "w or out is NULL");
  UNIFUR_HIP(launch_lora_merge(w, lora->a, lora->b, (int)lora->rank, lora->scaling, d_in, d_out, out,
                               static_cast<hipStream_t>(stream)));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_stripe_weight(const unifur_nf4_weight* src, uint8_t* dst_packed, void* dst_scales, void* stream) {
  if (int r = check_weight(src, "src")) return r;
  UNIFUR_ARG(src->layout == UNIFUR_NF4_LAYOUT_ROW_MAJOR, "stripe_weight takes a row-major weight");
  UNIFUR_ARG(src->d_out % 64 == 0, "the striped layout needs d_out % 64 == 0");
  UNIFUR_ARG(dst_packed && dst_scales, "dst_packed or dst_scales is NULL");
  UNIFUR_ARG(aligned_to(src->packed, 8) && aligned_to(dst_packed, 8), "packed codes must be 8-byte aligned");
  const bool dq = src->scales.kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  UNIFUR_HIP(launch_stripe_codes(src->packed, dst_packed, src->d_in, src->d_out, true, st));
  UNIFUR_HIP(launch_stripe_scales(dq ? (const void*)src->scales.dq_codes : (const void*)src->scales.absmax,
                                  dst_scales, src->d_in, src->d_out, dq, true, st));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_unstripe_weight(const unifur_nf4_weight* src, uint8_t* dst_packed, void* dst_scales, void* stream) {
  if (int r = check_weight(src, "src")) return r;
  UNIFUR_ARG(src->layout == UNIFUR_NF4_LAYOUT_STRIPED, "unstripe_weight takes a striped weight");
  UNIFUR_ARG(dst_packed && dst_scales, "dst_packed or dst_scales is NULL");
  UNIFUR_ARG(aligned_to(dst_packed, 8), "packed codes must be 8-byte aligned");
  const bool dq = src->scales.kind == UNIFUR_NF4_SCALES_DOUBLE_QUANTIZED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  UNIFUR_HIP(launch_stripe_codes(src->packed, dst_packed, src->d_in, src->d_out, false, st));
  UNIFUR_HIP(launch_stripe_scales(dq ? (const void*)src->scales.dq_codes : (const void*)src->scales.absmax,
                                  dst_scales, src->d_in, src->d_out, dq, false, st));
  return UNIFUR_NF4_OK;
}

int unifur_nf4_swiglu_forward(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* gate,
                              const unifur_nf4_weight* up, const unifur_nf4_weight* down, void* y, int y_dtype,
                              void* workspace, uint64_t workspace_bytes, void* stream) {
  return run_swiglu(x, x_dtype, rows, gate, up, down, y, y_dtype, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

}  // extern "C"
