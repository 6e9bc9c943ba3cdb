// Plain bf16 linears y[M, N] = x[M, K] . w[N, K]^T (fp32 accumulation, bf16 output) through
// hipBLASLt: the query and output projections of the memory readout (lngram_v2.py:1115-1118,
// :1354-1357), which carry no fused epilogue.  The router (sign-pack epilogue) and the output
// projection with row statistics keep the hand-written MFMA kernels of gemm.hip.
//
// In hipBLASLt's column-major terms y^T[N, M] = op(w) . x^T with w stored [K, N] (transposed)
// and x stored [K, M].  One handle per device and one matmul plan per (device, M, N, K) are made
// on first use (host-side state, guarded by a mutex) and reused; the GEMM runs without workspace.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "common.h"

namespace lng {

namespace {

struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

std::mutex g_lt_mu;
std::map<int, hipblasLtHandle_t> g_lt_handles;
std::map<std::tuple<int, int64_t, int64_t, int64_t>, LtPlan> g_lt_plans;

// Plan for the current device (nullptr when hipBLASLt offers no algorithm for the shape).
const LtPlan* lt_plan(hipblasLtHandle_t* handle, int64_t M, int64_t N, int64_t K) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> g(g_lt_mu);
  auto hi = g_lt_handles.find(dev);
  if (hi == g_lt_handles.end()) {
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return nullptr;
    hi = g_lt_handles.emplace(dev, h).first;
  }
  *handle = hi->second;
  const auto key = std::make_tuple(dev, M, N, K);
  auto pi = g_lt_plans.find(key);
  if (pi != g_lt_plans.end()) return pi->second.ok ? &pi->second : nullptr;
  LtPlan p;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
                HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
                HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, K, M, K) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_16BF, N, M, N) == HIPBLAS_STATUS_SUCCESS;
  if (ok) {
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    const uint64_t ws = 0;
    ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) ==
             HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulAlgoGetHeuristic(hi->second, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, res, &n) ==
             HIPBLAS_STATUS_SUCCESS &&
         n > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS;
    if (ok) p.algo = res[0].algo;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  }
  if (!ok) {  // no plan for this shape: keep the verdict, release the descriptors
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    for (hipblasLtMatrixLayout_t l : {p.la, p.lb, p.lc})
      if (l) hipblasLtMatrixLayoutDestroy(l);
    p.desc = nullptr;
    p.la = p.lb = p.lc = nullptr;
  }
  p.ok = ok;
  auto& slot = g_lt_plans[key] = p;
  return ok ? &slot : nullptr;
}

}  // namespace

// Returns LNG_OK when hipBLASLt ran the GEMM, LNG_E_ARG (no message) when it has no plan for the
// shape (the caller then runs its own kernel), LNG_E_HIP when the launch failed.
int linear_bf16_lt(const void* x, const void* w, int64_t M, int64_t N, int64_t K, void* y, hipStream_t s) {
  hipblasLtHandle_t h = nullptr;
  const LtPlan* p = lt_plan(&h, M, N, K);
  if (!p) return LNG_E_ARG;
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t st = hipblasLtMatmul(h, p->desc, &alpha, w, p->la, x, p->lb, &beta, y, p->lc, y, p->lc,
                                             &p->algo, nullptr, 0, s);
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(LNG_E_HIP, "linear: hipBLASLt matmul failed");
  return LNG_OK;
}

}  // namespace lng
