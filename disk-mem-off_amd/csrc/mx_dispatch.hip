// Token -> expert dispatch: histogram, prefix sums, expert-sorted row order.
//
// Reference: offload_runtime/executors/glm4_moe.py:206-215 and qwen3_next.py:297-305 —
// the active set is set(topk_indices) and each expert e gathers h[token_mask] rows in
// ascending token order.  This kernel produces the same grouping as a stable counting
// sort of the T*k (token, slot) pairs by expert id:
//   counts[e], offsets[e]      histogram and its exclusive prefix
//   sorted_tok[r], sorted_w[r] token and routing weight of expert-sorted row r
//   pair_pos[t*k + j]          row of pair (t, j)
//   groups                     shared expert first (rows T*k .. T*k+T-1), then the active
//                              routed experts in ascending id
//   m-tiles                    every group cut into m_blk-row tiles, in group order
// Everything is integer work in one workgroup; per-wave token ranges are ranked with a
// per-wave 64-bit LDS mask per expert, so the order is deterministic (no atomics decide
// a position).
#include "mx_common.h"
#include "mx_internal.h"

#include "mx_dispatch_dev.h"

__global__ __launch_bounds__(512) void k_dispatch(
    const int* __restrict__ ids, const float* __restrict__ tw, const float* __restrict__ shw,
    int T, int k, int E, int has_shared, int m_blk, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ sorted_tok, float* __restrict__ sorted_w,
    int* __restrict__ pair_pos, int* __restrict__ g_expert, int* __restrict__ g_start,
    int* __restrict__ g_count, int* __restrict__ n_groups, int* __restrict__ mt_group,
    int* __restrict__ mt_row0, int* __restrict__ n_mtiles) {
  extern __shared__ __align__(16) unsigned char smem[];
  mx_dispatch_block(smem, ids, tw, shw, T, k, E, has_shared, m_blk, counts, offsets, sorted_tok,
                    sorted_w, pair_pos, g_expert, g_start, g_count, n_groups, mt_group, mt_row0,
                    n_mtiles);
}


int mx_max_mtiles(int tokens, int top_k, int n_experts, int has_shared, int m_blk) {
  const long pairs = (long)tokens * top_k;
  long routed = pairs / m_blk + (pairs < n_experts ? pairs : n_experts);
  long shared = has_shared ? (tokens + m_blk - 1) / m_blk : 0;
  long total = routed + shared;
  return (int)(total > 0 ? total : 1);
}

extern "C" int mx_dispatch(const int32_t* topk_ids, const float* topk_w, const float* shared_w,
                           int32_t tokens, int32_t top_k, int32_t n_experts, int32_t has_shared,
                           int32_t m_blk, int32_t* counts, int32_t* offsets, int32_t* sorted_tok,
                           float* sorted_w, int32_t* pair_pos, int32_t* g_expert,
                           int32_t* g_start, int32_t* g_count, int32_t* n_groups,
                           int32_t* mt_group, int32_t* mt_row0, int32_t* n_mtiles, void* stream) {
  if (!topk_ids || !topk_w || !counts || !offsets || !sorted_tok || !sorted_w || !pair_pos ||
      !g_expert || !g_start || !g_count || !n_groups || !mt_group || !mt_row0 || !n_mtiles)
    return MX_ERR_INVALID;
  if (tokens < 0 || top_k < 1 || n_experts < 1 || m_blk < 1) return MX_ERR_INVALID;
  if (n_experts > 2048) return MX_ERR_UNSUPPORTED;
  if ((long)tokens * top_k > (1l << 30)) return MX_ERR_UNSUPPORTED;
  int nw = 8;
  while (nw > 1 && mx_dispatch_lds_bytes(nw, n_experts) > 60 * 1024) nw >>= 1;
  const size_t lds = mx_dispatch_lds_bytes(nw, n_experts);
  if (lds > 60 * 1024) return MX_ERR_UNSUPPORTED;
  mx_clear_error();
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(nw * 64), lds, (hipStream_t)stream, topk_ids,
                     topk_w, shared_w, (int)tokens, (int)top_k, (int)n_experts, (int)has_shared,
                     (int)m_blk, counts, offsets, sorted_tok, sorted_w, pair_pos, g_expert,
                     g_start, g_count, n_groups, mt_group, mt_row0, n_mtiles);
  return mx_launch_status();
}
