// Plain bf16 prefill GEMMs on hipBLASLt: y[M, N] = x[M, K] W[N, K]^T (+ bias),
// fp32 accumulation, one rounding to bf16 (bias added before it, as
// F.linear's addmm does, fused.py:58). Not the product path: the prompt
// GEMMs run on the library's own MFMA kernels, and these calls happen only
// when MINITP_GEMM=blaslt is set in the environment, as a comparison for the
// benchmark. Used only for prompt-sized M and
// never while the stream is being captured: the library's split-K
// algorithms may record memsets, which a captured decode graph must not
// hold. Residual adds stay outside (a separate rounded add, the reference's
// order), so the callers pass a temporary output.
//
// The hipBLASLt that serves the calls is whichever the process loaded first
// (a PyTorch process brings its own); a shape it has no solution for comes
// back MINITP_ERR_UNSUPPORTED and runs on launch_gemm.
//
// Algorithm choice: the first call of a shape asks the heuristic for up to
// TUNE_CANDIDATES algorithms, times each on the call's own operands (one
// warm run, then TUNE_REPS runs between two events, the stream synchronized)
// and keeps the fastest; heuristic rank 0 stays unless another is at least
// TUNE_MARGIN faster. The candidates compute the same product with different
// tilings and K splits, so results may differ between processes in the last
// bf16 bit. MINITP_BLASLT_TUNE=0 in the environment keeps rank 0 always.
//
// Row-major y = x W^T is the column-major product y^T = W^T' x^T': A = W
// stored K x N (ld K) used transposed, B = x stored K x M (ld ldx), D = y
// stored N x M (ld ldy); the bias is per row of D.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <map>
#include <vector>
#include <mutex>
#include <string>
#include <tuple>

#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

constexpr int TUNE_CANDIDATES = 8;
constexpr int TUNE_REPS = 2;
constexpr float TUNE_MARGIN = 0.03f;

}  // namespace

bool blaslt_requested() {
  static const bool on = [] {
    const char* v = getenv("MINITP_GEMM");
    return v != nullptr && std::string(v) == "blaslt";
  }();
  return on;
}

namespace {

bool tune_enabled() {
  static const bool on = [] {
    const char* v = getenv("MINITP_BLASLT_TUNE");
    return v == nullptr || v[0] != '0';
  }();
  return on;
}

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

using Key = std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t, bool, int64_t>;

struct Lt {
  std::mutex mu;
  std::map<int, hipblasLtHandle_t> handles;  // per device
  std::map<Key, Plan> plans;
};

Lt& lt() {
  static Lt* s = new Lt();  // lives until the process ends (handles outlive static destructors)
  return *s;
}

// Descriptors of y = x W^T (+ bias) and the heuristic's candidates that fit
// the workspace, best-ranked first.
bool build_plan(hipblasLtHandle_t h, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, bool bias,
                int64_t ws_bytes, Plan& p, std::vector<hipblasLtMatmulAlgo_t>& cands) {
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN));
  if (bias) {
    const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bt = HIP_R_16BF;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
  }
  if (hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, (uint64_t)K, (uint64_t)N, K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, (uint64_t)K, (uint64_t)M, ldx) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.ld, HIP_R_16BF, (uint64_t)N, (uint64_t)M, ldy) != HIPBLAS_STATUS_SUCCESS)
    return false;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
  const uint64_t wsb = (uint64_t)ws_bytes;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
  hipblasLtMatmulHeuristicResult_t res[TUNE_CANDIDATES] = {};
  int count = 0;
  const hipblasStatus_t s = hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.ld, p.ld, pref,
                                                            tune_enabled() ? TUNE_CANDIDATES : 1, res, &count);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (s != HIPBLAS_STATUS_SUCCESS) return false;
  for (int i = 0; i < count && i < TUNE_CANDIDATES; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= (size_t)ws_bytes)
      cands.push_back(res[i].algo);
  if (cands.empty()) return false;
  p.algo = cands[0];
  return true;
}

// Mean time of TUNE_REPS runs of one candidate after a warm run, or a
// negative value when the library refuses it for these operands.
float time_algo(hipblasLtHandle_t h, Plan& p, const hipblasLtMatmulAlgo_t& algo, const void* x, const void* w,
                void* y, void* ws, int64_t ws_bytes, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const float alpha = 1.f, beta = 0.f;
  auto run = [&] {
    return hipblasLtMatmul(h, p.desc, &alpha, w, p.la, x, p.lb, &beta, y, p.ld, y, p.ld, &algo, ws,
                           (size_t)ws_bytes, st) == HIPBLAS_STATUS_SUCCESS;
  };
  if (!run()) return -1.f;
  if (hipEventRecord(e0, st) != hipSuccess) return -1.f;
  for (int r = 0; r < TUNE_REPS; ++r)
    if (!run()) return -1.f;
  float ms = -1.f;
  if (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
      hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
    return -1.f;
  return ms / TUNE_REPS;
}

// Keeps the fastest candidate (rank 0 unless another beats it by the margin).
void tune_plan(hipblasLtHandle_t h, Plan& p, const std::vector<hipblasLtMatmulAlgo_t>& cands, const void* x,
               const void* w, void* y, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (cands.size() < 2) return;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0) (void)hipEventDestroy(e0);
    (void)hipGetLastError();
    return;
  }
  const float base = time_algo(h, p, cands[0], x, w, y, ws, ws_bytes, st, e0, e1);
  float best = base;
  size_t pick = 0;
  for (size_t i = 1; base > 0.f && i < cands.size(); ++i) {
    const float t = time_algo(h, p, cands[i], x, w, y, ws, ws_bytes, st, e0, e1);
    if (t > 0.f && t < best) {
      best = t;
      pick = i;
    }
  }
  if (pick != 0 && best < base * (1.f - TUNE_MARGIN)) p.algo = cands[pick];
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipGetLastError();
}

}  // namespace

int blaslt_linear_bf16(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* bias, void* y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws, int64_t ws_bytes) {
  if (M <= 0 || N <= 0 || K <= 0) return MINITP_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return MINITP_ERR_UNSUPPORTED;
  int dev = 0;
  MINITP_RETURN_HIP(hipGetDevice(&dev));
  Lt& L = lt();
  std::lock_guard<std::mutex> lock(L.mu);
  auto hit = L.handles.find(dev);
  if (hit == L.handles.end()) {
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) h = nullptr;
    hit = L.handles.emplace(dev, h).first;
  }
  hipblasLtHandle_t h = hit->second;
  if (h == nullptr) return MINITP_ERR_UNSUPPORTED;
  const Key key{dev, M, N, K, ldx, ldy, bias != nullptr, ws_bytes};
  auto it = L.plans.find(key);
  const bool fresh = it == L.plans.end();
  std::vector<hipblasLtMatmulAlgo_t> cands;
  if (fresh) {
    Plan p;
    p.ok = build_plan(h, M, N, K, ldx, ldy, bias != nullptr, ws_bytes, p, cands);
    it = L.plans.emplace(key, p).first;
  }
  Plan& p = it->second;
  if (!p.ok) return MINITP_ERR_UNSUPPORTED;
  if (bias != nullptr)
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
  if (fresh && tune_enabled()) tune_plan(h, p, cands, x, w, y, ws, ws_bytes, st);
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t s = hipblasLtMatmul(h, p.desc, &alpha, w, p.la, x, p.lb, &beta, y, p.ld, y, p.ld, &p.algo,
                                            ws, (size_t)ws_bytes, st);
  if (s != HIPBLAS_STATUS_SUCCESS) {
    set_error("hipblasLtMatmul failed (status %d) for M=%lld N=%lld K=%lld", (int)s, (long long)M, (long long)N,
              (long long)K);
    return MINITP_ERR_HIP;
  }
  return MINITP_OK;
}

}  // namespace minitp
