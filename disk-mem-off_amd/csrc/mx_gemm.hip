// Dense projections of the attention blocks: y[T, N] = a[T, K] W^T on the single-group
// down-projection kernels of the MoE experts (short inputs, and int8 / fp32 weights at any
// length) or on the dense fp16 MFMA GEMM (mx_gemm_f16, long inputs with fp16 weights).
#include "mx_common.h"
#include "mx_internal.h"

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
  return mx_align_up((size_t)n_ent * sizeof(MxExpertPtrs), 256) + 256 +
         2 * mx_align_up(n_mt * 4, 256) + mx_align_up((size_t)Tn * 4, 256);
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
  if (mx_dense_on_gemm(wdt, T, K)) {
    const MxGemmSeg g{wmat, y, N, N};
    return mx_gemm_f16(a, T, K, &g, 1, s);
  }
  const MxDenseTables tab{w.tabs + 0, w.tabs + 1, w.tabs + 2, w.mt_group, w.mt_row0,
                          w.tabs + 3, w.ones, w.m_blk};
  return mx_dense_linear(wdt, 0, w.entries + ent, tab, T, N, K, a, y, s);
}
