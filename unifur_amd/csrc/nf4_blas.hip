// nf4_blas.hip -- the plain bf16 GEMMs of the prefill and backward paths,
// through hipBLASLt.
//
// One row-major product in hipBLASLt's column-major terms (a row-major
// [R][C] array is the column-major C x R matrix with leading dimension C):
//   Y[M][N] = X[M][K] Wt[N][K]^T (+ bias): D (N x M, ld N) =
//             op_T(Wt as K x N, ld K) * (X as K x M, ld K) -- the "TN" form.
// The forward takes it with Wt the weight expanded transposed; the
// backward's dX[M][K] = dY[M][N] E[K][N]^T takes it with E the weight
// expanded in its own [K][N] orientation (as an "NN" product of dY and the
// transposed expansion the same shape ran 62.5 us against 53-54 us for the
// TN kernels, 2048 x 4096 x 4096, every candidate of both forms timed).
// bf16 operands, f32 accumulation (HIPBLAS_COMPUTE_32F), alpha 1, beta 0,
// the bias added by the library's epilogue.
//
// The library's heuristic ranks candidates without running them and its
// first choice is often not the fastest on this part, so the first call of a
// shape on a device times the candidates it returns (on the caller's
// stream) and keeps the fastest.
#include "nf4_expand.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace unifur {
namespace {

constexpr int kMaxDevices = 64;
// The first call of a shape times this many heuristic candidates, each over
// kTimedRuns launches after one warm-up, and keeps the fastest.  Eight
// candidates timed over three runs left the backward's dX product
// (2048 x 4096 x 4096, then an NN product) at 111 us; thirty-two over twelve
// found a 105 us kernel.  The search costs about 25 ms once per shape.
constexpr int kCandidates = 32;
constexpr int kTimedRuns = 12;

// One product in column-major terms: D (m x n) = op(A) op(B), op(A) m x k.
struct Shape {
  bool ta, tb;
  int m, n, k, lda, ldb, ldd;
};

struct Key {
  int dev;
  Shape s;
  bool y_bf16, bias;
  bool operator<(const Key& o) const {
    return std::tie(dev, s.ta, s.tb, s.m, s.n, s.k, s.lda, s.ldb, s.ldd, y_bf16, bias) <
           std::tie(o.dev, o.s.ta, o.s.tb, o.s.m, o.s.n, o.s.k, o.s.lda, o.s.ldb, o.s.ldd, o.y_bf16, o.bias);
  }
};

struct State {
  std::mutex mu;
  hipblasLtHandle_t handle[kMaxDevices] = {};
  std::map<Key, hipblasLtMatmulAlgo_t> tuned;
};

State& state() {
  static State s;
  return s;
}

hipError_t to_hip(hipblasStatus_t s) {
  switch (s) {
    case HIPBLAS_STATUS_SUCCESS: return hipSuccess;
    case HIPBLAS_STATUS_NOT_SUPPORTED: return hipErrorNotSupported;
    case HIPBLAS_STATUS_INVALID_VALUE: return hipErrorInvalidValue;
    case HIPBLAS_STATUS_ALLOC_FAILED: return hipErrorOutOfMemory;
    default: return hipErrorUnknown;
  }
}

#define BLAS_TRY(expr)                                   \
  do {                                                   \
    const hipblasStatus_t st_ = (expr);                  \
    if (st_ != HIPBLAS_STATUS_SUCCESS) return to_hip(st_); \
  } while (0)
#define HIP_TRY(expr)                  \
  do {                                 \
    const hipError_t e_ = (expr);      \
    if (e_ != hipSuccess) return e_;   \
  } while (0)

// The descriptors of one product (they hold the bias pointer, so each call
// builds its own).
struct Desc {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  ~Desc() {
    if (d) hipblasLtMatrixLayoutDestroy(d);
    if (b) hipblasLtMatrixLayoutDestroy(b);
    if (a) hipblasLtMatrixLayoutDestroy(a);
    if (op) hipblasLtMatmulDescDestroy(op);
  }
  hipblasStatus_t make(const Shape& sh, const float* bias, bool y_bf16) {
    hipblasStatus_t s = hipblasLtMatmulDescCreate(&op, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (s != HIPBLAS_STATUS_SUCCESS) return s;
    const hipblasOperation_t ta = sh.ta ? HIPBLAS_OP_T : HIPBLAS_OP_N, tb = sh.tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    if ((s = hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)))) return s;
    if ((s = hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)))) return s;
    if (bias) {
      const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
      const hipDataType bt = HIP_R_32F;
      if ((s = hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)))) return s;
      if ((s = hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)))) return s;
      if ((s = hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)))) return s;
    }
    // stored shapes: A is m x k (k x m when transposed), B k x n (n x k)
    if ((s = hipblasLtMatrixLayoutCreate(&a, HIP_R_16BF, sh.ta ? sh.k : sh.m, sh.ta ? sh.m : sh.k, sh.lda))) return s;
    if ((s = hipblasLtMatrixLayoutCreate(&b, HIP_R_16BF, sh.tb ? sh.n : sh.k, sh.tb ? sh.k : sh.n, sh.ldb))) return s;
    return hipblasLtMatrixLayoutCreate(&d, y_bf16 ? HIP_R_16BF : HIP_R_32F, sh.m, sh.n, sh.ldd);
  }
};

hipError_t handle_for(int dev, bool capturing, hipblasLtHandle_t* out) {
  State& st = state();
  std::lock_guard<std::mutex> lock(st.mu);
  if (!st.handle[dev]) {
    // creating a handle allocates device memory: not under stream capture
    if (capturing) return hipErrorStreamCaptureUnsupported;
    BLAS_TRY(hipblasLtCreate(&st.handle[dev]));
  }
  *out = st.handle[dev];
  return hipSuccess;
}

hipError_t time_candidate(hipblasLtHandle_t h, const Desc& dsc, const hipblasLtMatmulAlgo_t& algo, const void* A,
                          const void* B, void* y, void* ws, size_t ws_bytes, hipStream_t stream, float* ms) {
  const float alpha = 1.0f, beta = 0.0f;
  auto run = [&]() {
    return hipblasLtMatmul(h, dsc.op, &alpha, A, dsc.a, B, dsc.b, &beta, y, dsc.d, y, dsc.d, &algo, ws, ws_bytes,
                           stream);
  };
  BLAS_TRY(run());
  hipEvent_t e0 = nullptr, e1 = nullptr;
  HIP_TRY(hipEventCreate(&e0));
  hipError_t e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipEventRecord(e0, stream);
  for (int i = 0; i < kTimedRuns && e == hipSuccess; ++i) e = to_hip(run());
  if (e == hipSuccess) e = hipEventRecord(e1, stream);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, e0, e1);
  (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  return e;
}

}  // namespace

namespace {

hipError_t gemm_cm(const Shape& sh, const void* A, const void* B, const float* bias, void* y, bool y_bf16, void* ws,
                   size_t ws_bytes, hipStream_t stream) {
  if (sh.m <= 0 || sh.n <= 0 || sh.k <= 0 || !A || !B || !y) return hipErrorInvalidValue;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(stream, &cap));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  hipblasLtHandle_t h = nullptr;
  HIP_TRY(handle_for(dev, capturing, &h));

  Desc dsc;
  BLAS_TRY(dsc.make(sh, bias, y_bf16));
  const Key key{dev, sh, y_bf16, bias != nullptr};
  hipblasLtMatmulAlgo_t algo{};
  bool have = false;
  {
    State& st = state();
    std::lock_guard<std::mutex> lock(st.mu);
    auto it = st.tuned.find(key);
    if (it != st.tuned.end()) {
      algo = it->second;
      have = true;
    }
  }
  if (!have) {
    hipblasLtMatmulPreference_t pref = nullptr;
    BLAS_TRY(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t limit = ws_bytes;
    hipblasStatus_t s =
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &limit, sizeof(limit));
    hipblasLtMatmulHeuristicResult_t res[kCandidates] = {};
    int n = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
      s = hipblasLtMatmulAlgoGetHeuristic(h, dsc.op, dsc.a, dsc.b, dsc.d, dsc.d, pref, kCandidates, res, &n);
    hipblasLtMatmulPreferenceDestroy(pref);
    BLAS_TRY(s);
    if (n <= 0) return hipErrorNotSupported;
    int best = 0;
    if (!capturing) {
      float best_ms = -1.0f;
      for (int i = 0; i < n; ++i) {
        if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > ws_bytes) continue;
        float ms = 0.0f;
        if (time_candidate(h, dsc, res[i].algo, A, B, y, ws, ws_bytes, stream, &ms) != hipSuccess) continue;
        if (best_ms < 0.0f || ms < best_ms) {
          best_ms = ms;
          best = i;
        }
      }
      if (best_ms < 0.0f) return hipErrorNotSupported;
      State& st = state();
      std::lock_guard<std::mutex> lock(st.mu);
      st.tuned[key] = res[best].algo;
    }
    algo = res[best].algo;
  }
  const float alpha = 1.0f, beta = 0.0f;
  BLAS_TRY(hipblasLtMatmul(h, dsc.op, &alpha, A, dsc.a, B, dsc.b, &beta, y, dsc.d, y, dsc.d, &algo, ws, ws_bytes,
                           stream));
  return hipSuccess;
}

}  // namespace

hipError_t blas_gemm_xwt(const uint16_t* x, const uint16_t* wt, const float* bias, int M, int N, int K, void* y,
                         bool y_bf16, void* ws, size_t ws_bytes, hipStream_t stream) {
  return blas_gemm_xwt_ld(x, wt, bias, M, N, K, y, N, y_bf16, ws, ws_bytes, stream);
}

hipError_t blas_gemm_xwt_ld(const uint16_t* x, const uint16_t* wt, const float* bias, int M, int N, int K, void* y,
                            int ldy, bool y_bf16, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (ldy < N) return hipErrorInvalidValue;
  const Shape sh{true, false, N, M, K, K, K, ldy};
  return gemm_cm(sh, wt, x, bias, y, y_bf16, ws, ws_bytes, stream);
}

bool blas_gemm_xwt_tuned(int M, int N, int K, bool y_bf16) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  const Shape sh{true, false, N, M, K, K, K, N};
  State& st = state();
  std::lock_guard<std::mutex> lock(st.mu);
  return st.tuned.count(Key{dev, sh, y_bf16, false}) != 0;
}

}  // namespace unifur
