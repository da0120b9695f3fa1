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

// ------------------------------------------------------------------------------------
// Dense projections of the attention blocks: y[T, N] = a[T, K] W^T, on hipBLASLt for long
// inputs (falling back to the expert kernels when the library has no algorithm for the
// shape) and on the single-group down-projection kernels otherwise.
// ------------------------------------------------------------------------------------
namespace {

__global__ __launch_bounds__(256) void k_dense_setup(int T, int m_blk, int n_mt,
                                                     MxDenseEntries ents, int n_ent,
                                                     MxExpertPtrs* __restrict__ entries,
                                                     int* __restrict__ tabs,
                                                     int* __restrict__ mt_group,
                                                     int* __restrict__ mt_row0,
                                                     float* __restrict__ ones) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n_ent) entries[i] = ents.e[i];
  if (i == 0) {
    tabs[0] = 0;  // g_expert
    tabs[1] = 0;  // g_start
    tabs[2] = T;  // g_count
    tabs[3] = n_mt;
  }
  if (i < n_mt) {
    mt_group[i] = 0;
    mt_row0[i] = i * m_blk;
  }
  if (i < T) ones[i] = 1.f;
}

}  // namespace

size_t mx_dense_work_bytes(int T, int weight_dtype, int n_ent) {
  const int Tn = T > 0 ? T : 1;
  const int m_blk = mx_m_blk_for(Tn, weight_dtype);
  const size_t n_mt = (size_t)mx_ceil_div(Tn, m_blk);
  size_t b = mx_align_up((size_t)n_ent * sizeof(MxExpertPtrs), 256) + 256 +
             2 * mx_align_up(n_mt * 4, 256) + mx_align_up((size_t)Tn * 4, 256);
  if (Tn >= MX_DENSE_BLAS_MIN_TOKENS && weight_dtype != MX_DT_I8) b += mx_gemm_workspace_bytes();
  return b;
}

void mx_dense_work_carve(char* base, int T, int weight_dtype, int n_ent, MxDenseWork* w) {
  const int Tn = T > 0 ? T : 1;
  w->m_blk = mx_m_blk_for(Tn, weight_dtype);
  w->n_mt = mx_ceil_div(Tn, w->m_blk);
  w->n_ent = n_ent;
  char* p = base;
  w->entries = (MxExpertPtrs*)p;
  p += mx_align_up((size_t)n_ent * sizeof(MxExpertPtrs), 256);
  w->tabs = (int*)p;
  p += 256;
  w->mt_group = (int*)p;
  p += mx_align_up((size_t)w->n_mt * 4, 256);
  w->mt_row0 = (int*)p;
  p += mx_align_up((size_t)w->n_mt * 4, 256);
  w->ones = (float*)p;
  p += mx_align_up((size_t)Tn * 4, 256);
  const bool blas = Tn >= MX_DENSE_BLAS_MIN_TOKENS && weight_dtype != MX_DT_I8;
  w->blas_ws = blas ? (void*)p : nullptr;
  w->blas_ws_bytes = blas ? mx_gemm_workspace_bytes() : 0;
}

int mx_dense_setup(const MxDenseWork& w, const MxDenseEntries& ents, int T, hipStream_t s) {
  if (w.n_ent > MX_DENSE_MAX_ENT) return MX_ERR_INVALID;
  int nth = T > w.n_mt ? T : w.n_mt;
  if (w.n_ent > nth) nth = w.n_ent;
  mx_clear_error();
  hipLaunchKernelGGL(k_dense_setup, dim3(mx_ceil_div(nth, 256)), dim3(256), 0, s, T, w.m_blk,
                     w.n_mt, ents, w.n_ent, w.entries, w.tabs, w.mt_group, w.mt_row0, w.ones);
  return mx_launch_status();
}

int mx_project(const MxDenseWork& w, int ent, int wdt, const void* wmat, int T, int N, int K,
               const void* a, float* y, hipStream_t s) {
  if (ent < 0 || ent >= w.n_ent) return MX_ERR_INVALID;
  if (w.blas_ws && T >= MX_DENSE_BLAS_MIN_TOKENS && wdt != MX_DT_I8) {
    const int rc = mx_gemm_wt(wdt, a, wmat, y, T, N, K, w.blas_ws, w.blas_ws_bytes, s);
    if (rc != MX_ERR_UNSUPPORTED) return rc;
  }
  const MxDenseTables tab{w.tabs + 0, w.tabs + 1, w.tabs + 2, w.mt_group, w.mt_row0,
                          w.tabs + 3, w.ones, w.m_blk};
  return mx_dense_linear(wdt, 0, w.entries + ent, tab, T, N, K, a, y, s);
}
