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
#include "nf4_codec.hpp"
#include "nf4_gemm.hpp"
#include "nf4_generic.hpp"
#include "nf4_gemv.hpp"

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

int check_weight(const unifur_nf4_weight* w, const char* name) {
  UNIFUR_ARG(w != nullptr, std::string(name) + " weight is NULL");
  UNIFUR_ARG(w->packed != nullptr, std::string(name) + " packed codes are NULL");
  UNIFUR_ARG(w->d_in > 0 && w->d_out > 0, std::string(name) + " has a zero dimension");
  UNIFUR_ARG(w->d_in <= 0x7fffffffu && w->d_out <= 0x7fffffffu, std::string(name) + " dimension exceeds 2^31-1");
  return check_scales(&w->scales);
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
int internal_workspace(size_t bytes, hipStream_t stream, void** out) {
  int dev = 0;
  UNIFUR_HIP(hipGetDevice(&dev));
  WsCache& c = ws_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  auto& slot = c.buffers[{dev, stream}];
  if (slot.second < bytes) {
    if (slot.first) {
      UNIFUR_HIP(hipStreamSynchronize(stream));
      UNIFUR_HIP(hipFree(slot.first));
      slot = {nullptr, 0};
    }
    const size_t sz = align_up(bytes < (1u << 20) ? (1u << 20) : bytes);
    void* p = nullptr;
    UNIFUR_HIP(hipMalloc(&p, sz));
    UNIFUR_HIP(hipMemsetAsync(p, 0, sz, stream));
    slot = {p, sz};
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
struct Carver {
  size_t off = kCounterRegion;
  size_t take(size_t bytes) {
    size_t o = off;
    off += align_up(bytes);
    return o;
  }
};

// ------------------------------------------------------------- linear plans --

enum class LinearPath { kGemv, kMfma, kGeneric };

// The fused GEMV needs whole 64-blocks per weight row (d_out % 64 == 0),
// 16-byte aligned code rows and a weight that 32-bit buffer offsets reach
// (under 2 GiB of codes, 4 G values); every other shape takes the generic path.
bool gemv_layout_ok(uint64_t d_in, uint64_t d_out, const void* packed) {
  return d_out % 64 == 0 && (reinterpret_cast<uintptr_t>(packed) & 15u) == 0 && d_in * d_out / 2 < (1ull << 31);
}

struct LinearLayout {
  LinearPath path;
  GemvPlan gemv;
  size_t counters, partials, xa, xa_part, wf32, total;
};

// Decode-sized batches (<= 4 rows) take the fused GEMV; larger bf16 batches
// the MFMA GEMM; everything else the generic dequantize + f32 matmul.
LinearLayout plan_linear(uint64_t rows, uint64_t d_in, uint64_t d_out, uint32_t lora_rank, const void* packed,
                         int x_dtype, const void* x) {
  LinearLayout L{};
  Carver c;
  const bool gemv = rows <= (uint64_t)kGemvMaxRows && gemv_layout_ok(d_in, d_out, packed) &&
                    ceil_div_u64(d_out, 256) <= (uint64_t)kMaxCounters;
  const bool mfma = !gemv && x_dtype == UNIFUR_NF4_BF16 && gemv_layout_ok(d_in, d_out, packed) &&
                    rows <= 0x7fffffffu && d_in <= 0x7fffffffu && d_out <= 0x7fffffffu &&
                    gemm_supported((int)rows, (int)d_in, (int)d_out, x);
  if (gemv) {
    L.path = LinearPath::kGemv;
    const int n = (int)d_out;
    L.gemv = plan_gemv((int)rows, (int)d_in, &n, 1, false);
    L.counters = 0;
    L.partials = c.take(L.gemv.partial_count[0] * sizeof(float));
  } else if (mfma) {
    L.path = LinearPath::kMfma;
  } else {
    L.path = LinearPath::kGeneric;
    L.wf32 = c.take((size_t)d_in * d_out * sizeof(float));
  }
  const uint64_t xa_cols = L.path == LinearPath::kMfma && lora_rank ? (uint64_t)lora_pad((int)lora_rank) : lora_rank;
  L.xa = c.take((size_t)rows * xa_cols * sizeof(float));
  if (L.path == LinearPath::kMfma && lora_rank)
    L.xa_part = c.take(lora_xa_partial_floats((int)rows, (int)d_in, (int)lora_rank) * sizeof(float));
  L.total = c.off;
  return L;
}

template <typename T>
T* at(void* base, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

int run_linear(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w, const float* bias,
               const unifur_nf4_lora* lora, void* y, int y_dtype, void* workspace, uint64_t workspace_bytes,
               hipStream_t stream) {
  UNIFUR_ARG(valid_dtype(x_dtype) && valid_dtype(y_dtype), "dtype must be UNIFUR_NF4_F32 or UNIFUR_NF4_BF16");
  if (int r = check_weight(w, "linear")) return r;
  if (rows == 0) return UNIFUR_NF4_OK;
  UNIFUR_ARG(x != nullptr && y != nullptr, "x or y is NULL");
  UNIFUR_ARG(rows <= 0x7fffffffu, "rows exceeds 2^31-1");
  const uint32_t rank = lora ? lora->rank : 0;
  if (lora) {
    UNIFUR_ARG(lora->a != nullptr && lora->b != nullptr, "lora factors are NULL");
    UNIFUR_ARG(rank >= 1 && rank <= 64, "lora rank must be in [1, 64]");
  }
  const LinearLayout L = plan_linear(rows, w->d_in, w->d_out, rank, w->packed, x_dtype, x);
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  const bool xbf = x_dtype == UNIFUR_NF4_BF16;
  float* xa = nullptr;
  if (L.path == LinearPath::kMfma) {
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    if (lora) {
      xa = at<float>(ws, L.xa);
      UNIFUR_HIP(launch_lora_xa_bf16(xb, lora->a, (int)rows, (int)w->d_in, (int)rank, lora->scaling,
                                     at<float>(ws, L.xa_part), xa, stream));
    }
    UNIFUR_HIP(launch_gemm(xb, w->packed, to_scales(w->scales), (int)rows, (int)w->d_in, (int)w->d_out, bias, xa,
                           lora ? lora->b : nullptr, (int)rank, y, y_dtype == UNIFUR_NF4_BF16, stream));
    return UNIFUR_NF4_OK;
  }
  if (lora) {
    xa = at<float>(ws, L.xa);
    UNIFUR_HIP(launch_lora_xa(x, xbf, lora->a, (int)rows, (int)w->d_in, (int)rank, xa, stream));
  }
  if (L.path == LinearPath::kGemv) {
    GemvWeight gw{};
    gw.packed = w->packed;
    gw.scales = to_scales(w->scales);
    gw.d_out = (int)w->d_out;
    gw.y = y;
    gw.y_bf16 = y_dtype == UNIFUR_NF4_BF16;
    gw.bias = bias;
    gw.lora_xa = xa;
    gw.lora_b = lora ? lora->b : nullptr;
    gw.lora_rank = (int)rank;
    gw.lora_scaling = lora ? lora->scaling : 0.0f;
    gw.counters = at<unsigned>(ws, L.counters);
    gw.partials = at<float>(ws, L.partials);
    UNIFUR_HIP(launch_gemv(L.gemv, x, xbf, (int)rows, (int)w->d_in, &gw, 1, stream));
    return UNIFUR_NF4_OK;
  }
  // Generic: the reference's own sequence -- dequantize the whole weight to
  // f32 (bit-exact), then an f32 matmul.
  float* wf = at<float>(ws, L.wf32);
  UNIFUR_HIP(launch_dequantize(w->packed, to_scales(w->scales), (size_t)w->d_in * w->d_out, wf, false,
                               u32_aligned(w->packed), stream));
  Epilogue e{bias, xa, lora ? lora->b : nullptr, (int)rank, lora ? lora->scaling : 0.0f, y,
             y_dtype == UNIFUR_NF4_BF16};
  UNIFUR_HIP(launch_gemm_f32(x, xbf, wf, (int)rows, (int)w->d_in, (int)w->d_out, e, stream));
  return UNIFUR_NF4_OK;
}

// ------------------------------------------------------------- swiglu plans --

enum class MlpPath { kPairGemv, kGemv, kGeneric };

struct MlpLayout {
  MlpPath path;
  GemvPlan up_plan, down_plan;
  size_t counters, partials0, partials1, h, u, wf32, total;
};

MlpLayout plan_mlp(uint64_t rows, uint64_t hidden, uint64_t inter, const void* pg, const void* pu, const void* pd) {
  MlpLayout L{};
  Carver c;
  const bool layout = gemv_layout_ok(hidden, inter, pg) && gemv_layout_ok(hidden, inter, pu) &&
                      gemv_layout_ok(inter, hidden, pd) &&
                      ceil_div_u64(std::max(inter, hidden), 256) <= (uint64_t)kMaxCounters;
  if (layout && rows <= (uint64_t)kGemvMaxRows) {
    L.path = rows <= (uint64_t)kGemvPairMaxRows ? MlpPath::kPairGemv : MlpPath::kGemv;
    const int gi[2] = {(int)inter, (int)inter};
    const int hd = (int)hidden;
    L.up_plan = plan_gemv((int)rows, (int)hidden, gi, 2, L.path == MlpPath::kPairGemv);
    L.down_plan = plan_gemv((int)rows, (int)inter, &hd, 1, false);
    L.counters = 0;
    L.partials0 = c.take(std::max(L.up_plan.partial_count[0], L.down_plan.partial_count[0]) * sizeof(float));
    L.partials1 = c.take(L.up_plan.partial_count[1] * sizeof(float));
    L.h = c.take((size_t)rows * inter * sizeof(float));
    L.u = L.path == MlpPath::kGemv ? c.take((size_t)rows * inter * sizeof(float)) : 0;
  } else {
    L.path = MlpPath::kGeneric;
    L.wf32 = c.take((size_t)hidden * inter * sizeof(float));
    L.h = c.take((size_t)rows * inter * sizeof(float));
    L.u = c.take((size_t)rows * inter * sizeof(float));
  }
  L.total = c.off;
  return L;
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
  const MlpLayout L = plan_mlp(rows, hidden, inter, gate->packed, up->packed, down->packed);
  void* ws = nullptr;
  if (int r = resolve_workspace(workspace, workspace_bytes, L.total, stream, &ws)) return r;
  const bool xbf = x_dtype == UNIFUR_NF4_BF16;
  const bool ybf = y_dtype == UNIFUR_NF4_BF16;
  float* h = at<float>(ws, L.h);
  if (L.path == MlpPath::kPairGemv || L.path == MlpPath::kGemv) {
    unsigned* cnt = at<unsigned>(ws, L.counters);
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
  // Generic: three dequantize + f32 matmul linears and the elementwise middle.
  float* wf = at<float>(ws, L.wf32);
  float* u = at<float>(ws, L.u);
  const Epilogue none{};
  Epilogue eg = none, eu = none, ed = none;
  eg.y = h;
  eu.y = u;
  ed.y = y;
  ed.y_bf16 = ybf;
  UNIFUR_HIP(launch_dequantize(gate->packed, to_scales(gate->scales), hidden * inter, wf, false,
                               u32_aligned(gate->packed), stream));
  UNIFUR_HIP(launch_gemm_f32(x, xbf, wf, (int)rows, (int)hidden, (int)inter, eg, stream));
  UNIFUR_HIP(launch_dequantize(up->packed, to_scales(up->scales), hidden * inter, wf, false,
                               u32_aligned(up->packed), stream));
  UNIFUR_HIP(launch_gemm_f32(x, xbf, wf, (int)rows, (int)hidden, (int)inter, eu, stream));
  UNIFUR_HIP(launch_silu_mul(h, u, (size_t)rows * inter, h, stream));
  UNIFUR_HIP(launch_dequantize(down->packed, to_scales(down->scales), inter * hidden, wf, false,
                               u32_aligned(down->packed), stream));
  UNIFUR_HIP(launch_gemm_f32(h, false, wf, (int)rows, (int)inter, (int)hidden, ed, stream));
  return UNIFUR_NF4_OK;
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

uint64_t unifur_nf4_linear_workspace_size(uint64_t rows, uint64_t d_in, uint64_t d_out, int x_dtype,
                                          uint32_t lora_rank) {
  if (rows == 0 || d_in == 0 || d_out == 0) return 0;
  // sized for 16-byte-aligned buffers, as hipMalloc returns them; a call
  // with misaligned buffers may take the generic path, which needs more and
  // reports UNIFUR_NF4_ERR_WORKSPACE with the size when given less
  const void* aligned = reinterpret_cast<const void*>(uintptr_t{256});
  return plan_linear(rows, d_in, d_out, lora_rank, aligned, x_dtype, aligned).total;
}

int unifur_nf4_linear_forward(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w,
                              const float* bias, const unifur_nf4_lora* lora, void* y, int y_dtype, void* workspace,
                              uint64_t workspace_bytes, void* stream) {
  return run_linear(x, x_dtype, rows, w, bias, lora, y, y_dtype, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

int unifur_nf4_qlora_forward(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* w,
                             const unifur_nf4_lora* lora, void* y, int y_dtype, void* workspace,
                             uint64_t workspace_bytes, void* stream) {
  UNIFUR_ARG(lora != nullptr, "qlora_forward needs a lora adapter");
  return run_linear(x, x_dtype, rows, w, nullptr, lora, y, y_dtype, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

uint64_t unifur_nf4_swiglu_workspace_size(uint64_t rows, uint64_t hidden, uint64_t intermediate, int x_dtype) {
  (void)x_dtype;
  if (rows == 0 || hidden == 0 || intermediate == 0) return 0;
  const void* p = reinterpret_cast<const void*>(uintptr_t{256});
  return plan_mlp(rows, hidden, intermediate, p, p, p).total;
}

int unifur_nf4_swiglu_forward(const void* x, int x_dtype, uint64_t rows, const unifur_nf4_weight* gate,
                              const unifur_nf4_weight* up, const unifur_nf4_weight* down, void* y, int y_dtype,
                              void* workspace, uint64_t workspace_bytes, void* stream) {
  return run_swiglu(x, x_dtype, rows, gate, up, down, y, y_dtype, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream));
}

}  // extern "C"
