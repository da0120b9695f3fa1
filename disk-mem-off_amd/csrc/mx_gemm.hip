// Dense row-major products y[T, N] (fp32) = a[T, K] W[N, K]^T on hipBLASLt, for the plain
// library GEMMs of long inputs (the linear-attention projections at prefill sizes).  One
// hipBLASLt handle per device, created on first use and kept for the life of the process;
// per shape the matmul / layout descriptors and the heuristic's algorithm are cached, so a
// repeated call only launches.  The caller supplies the workspace.
//
// Column-major view: row-major W[N, K] is a K x N matrix (ld K), row-major a[T, K] is
// K x T (ld K) and row-major y[T, N] is N x T (ld N), so y^T = op_T(W) * a.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "mx_common.h"
#include "mx_internal.h"

namespace {

struct GemmPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo;
  bool ok = false;
};

constexpr int kMaxDevices = 64;
std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
std::map<std::tuple<int, int, int, int, int>, GemmPlan> g_plans;  // (dev, dtype, T, N, K)

int plan_for(int dev, int dtype, int T, int N, int K, size_t ws_bytes, GemmPlan** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (dev < 0 || dev >= kMaxDevices) return MX_ERR_UNSUPPORTED;
  if (!g_handle[dev] && hipblasLtCreate(&g_handle[dev]) != HIPBLAS_STATUS_SUCCESS)
    return MX_ERR_UNSUPPORTED;
  auto key = std::make_tuple(dev, dtype, T, N, K);
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    *out = &it->second;
    return it->second.ok ? MX_OK : MX_ERR_UNSUPPORTED;
  }
  GemmPlan& p = g_plans[key];
  *out = &p;
  const hipDataType ab = dtype == MX_DT_F16 ? HIP_R_16F : HIP_R_32F;
  hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  bool good = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
                  HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta,
                                              sizeof(ta)) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb,
                                              sizeof(tb)) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.la, ab, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.lb, ab, K, T, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, N, T, N) == HIPBLAS_STATUS_SUCCESS;
  if (good) {
    hipblasLtMatmulPreference_t pref = nullptr;
    uint64_t wmax = ws_bytes;
    hipblasLtMatmulHeuristicResult_t res[1];
    int count = 0;
    good = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                 &wmax, sizeof(wmax)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulAlgoGetHeuristic(g_handle[dev], p.desc, p.la, p.lb, p.lc, p.lc, pref, 1,
                                           res, &count) == HIPBLAS_STATUS_SUCCESS &&
           count > 0 && res[0].workspaceSize <= ws_bytes;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (good) p.algo = res[0].algo;
  }
  p.ok = good;
  return good ? MX_OK : MX_ERR_UNSUPPORTED;
}

}  // namespace

size_t mx_gemm_workspace_bytes() { return (size_t)32 << 20; }

int mx_gemm_wt(int dtype, const void* a, const void* w, float* y, int T, int N, int K, void* ws,
               size_t ws_bytes, hipStream_t s) {
  if (dtype != MX_DT_F16 && dtype != MX_DT_F32) return MX_ERR_UNSUPPORTED;
  if (!a || !w || !y || T <= 0 || N <= 0 || K <= 0) return MX_ERR_INVALID;
  int dev = 0;
  MX_TRY(mx_status(hipGetDevice(&dev)));
  GemmPlan* p = nullptr;
  MX_TRY(plan_for(dev, dtype, T, N, K, ws_bytes, &p));
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t st =
      hipblasLtMatmul(g_handle[dev], p->desc, &alpha, w, p->la, a, p->lb, &beta, y, p->lc, y,
                      p->lc, &p->algo, ws, ws_bytes, s);
  return st == HIPBLAS_STATUS_SUCCESS ? MX_OK : MX_ERR_UNSUPPORTED;
}
