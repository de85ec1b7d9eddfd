// Plain bf16 prefill GEMMs on hipBLASLt: y[M, N] = x[M, K] W[N, K]^T (+ bias),
// fp32 accumulation, one rounding to bf16 (bias added before it, as
// F.linear's addmm does, fused.py:58). Used only for prompt-sized M and
// never while the stream is being captured: the library's split-K
// algorithms may record memsets, which a captured decode graph must not
// hold. Residual adds stay outside (a separate rounded add, the reference's
// order), so the callers pass a temporary output.
//
// The hipBLASLt that serves the calls is whichever the process loaded first
// (a PyTorch process brings its own); a shape it has no solution for comes
// back MINITP_ERR_UNSUPPORTED and runs on launch_gemm.
//
// Row-major y = x W^T is the column-major product y^T = W^T' x^T': A = W
// stored K x N (ld K) used transposed, B = x stored K x M (ld ldx), D = y
// stored N x M (ld ldy); the bias is per row of D.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "common.h"
#include "kernels.h"

namespace minitp {

namespace {

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

bool build_plan(hipblasLtHandle_t h, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, bool bias,
                int64_t ws_bytes, Plan& p) {
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
  hipblasLtMatmulHeuristicResult_t res{};
  int count = 0;
  const hipblasStatus_t s =
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.ld, p.ld, pref, 1, &res, &count);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (s != HIPBLAS_STATUS_SUCCESS || count < 1 || res.state != HIPBLAS_STATUS_SUCCESS ||
      res.workspaceSize > (size_t)ws_bytes)
    return false;
  p.algo = res.algo;
  return true;
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
  if (it == L.plans.end()) {
    Plan p;
    p.ok = build_plan(h, M, N, K, ldx, ldy, bias != nullptr, ws_bytes, p);
    it = L.plans.emplace(key, p).first;
  }
  Plan& p = it->second;
  if (!p.ok) return MINITP_ERR_UNSUPPORTED;
  if (bias != nullptr)
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
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
