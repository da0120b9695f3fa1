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
  if (n_experts > 2048 || top_k > MX_DISPATCH_MAXK) return MX_ERR_UNSUPPORTED;
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

// ------------------------------------------------------------------------------------
// Chunked dispatch for large T: the same tables as k_dispatch, built by three launches.
//   1. k_dispatch_count (one block per chunk of DC_TOK tokens): per-wave 64-bit LDS masks
//      give each pair its stable rank inside the wave; a prefix over the chunk's 4 waves
//      turns it into the rank inside the chunk; per-chunk expert counts go to scratch.
//   2. k_dispatch_scan (one workgroup): per expert, exclusive prefix over chunks (chunk
//      bases, in place), totals, then the scans / offsets / groups / m-tiles of the
//      single-workgroup version.
//   3. k_dispatch_place (grid over pairs): row = offset[e] + chunk_base[c][e] + rank.
// The row order is identical to k_dispatch's (ascending token inside each expert).
// ------------------------------------------------------------------------------------
#define DC_TOK 256

__global__ __launch_bounds__(256) void k_dispatch_count(const int* __restrict__ ids, int T, int k,
                                                        int E, int* __restrict__ chunk_counts,
                                                        int* __restrict__ rank) {
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned long long* mask = (unsigned long long*)smem;  // [4][E]
  int* wcnt = (int*)(mask + 4 * (size_t)E);               // [4][E]
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < 4 * E; i += 256) wcnt[i] = 0;
  mx_lds_sync();
  const int t = c * DC_TOK + w * 64 + lane;
  const bool v = t < T;
  unsigned long long* wm = mask + (size_t)w * E;
  int* wc = wcnt + w * E;
  const unsigned long long below = (1ull << lane) - 1ull;
  int ev[MX_DISPATCH_MAXK];
#pragma unroll
  for (int j = 0; j < MX_DISPATCH_MAXK; ++j) {
    ev[j] = -1;
    if (j < k) {
      const int e = v ? ids[t * k + j] : -1;
      ev[j] = (unsigned)e < (unsigned)E ? e : -1;
    }
  }
#pragma unroll
  for (int j = 0; j < MX_DISPATCH_MAXK; ++j)
    if (j < k && ev[j] >= 0) wm[ev[j]] = 0ull;
  mx_lds_fence();
#pragma unroll
  for (int j = 0; j < MX_DISPATCH_MAXK; ++j)
    if (j < k && ev[j] >= 0) atomicOr(&wm[ev[j]], 1ull << lane);
  mx_lds_fence();
  unsigned long long mv[MX_DISPATCH_MAXK];
#pragma unroll
  for (int j = 0; j < MX_DISPATCH_MAXK; ++j) {
    mv[j] = 0ull;
    if (j < k && ev[j] >= 0) mv[j] = wm[ev[j]];
  }
  // One lane per (wave, expert) publishes the wave's count.
#pragma unroll
  for (int j = 0; j < MX_DISPATCH_MAXK; ++j)
    if (j < k && ev[j] >= 0 && (mv[j] & below) == 0ull) wc[ev[j]] = __popcll(mv[j]);
  mx_lds_sync();
  for (int e = tid; e < E; e += 256) {
    int run = 0;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const int n = wcnt[ww * E + e];
      wcnt[ww * E + e] = run;
      run += n;
    }
    chunk_counts[(size_t)c * E + e] = run;
  }
  mx_lds_sync();
#pragma unroll
  for (int j = 0; j < MX_DISPATCH_MAXK; ++j)
    if (j < k && ev[j] >= 0) rank[t * k + j] = wc[ev[j]] + __popcll(mv[j] & below);
}

__global__ __launch_bounds__(1024) void k_dispatch_scan(
    const float* __restrict__ shw, int T, int k, int E, int nch, int has_shared, int m_blk,
    int* __restrict__ chunk_counts, int* __restrict__ counts, int* __restrict__ offsets,
    int* __restrict__ sorted_tok, float* __restrict__ sorted_w, int* __restrict__ g_expert,
    int* __restrict__ g_start, int* __restrict__ g_count, int* __restrict__ n_groups,
    int* __restrict__ mt_group, int* __restrict__ mt_row0, int* __restrict__ n_mtiles) {
  extern __shared__ __align__(16) unsigned char smem[];
  int* tot = (int*)smem;
  int* off = tot + E;
  int* gid = off + E;
  int* mtb = gid + E;
  __shared__ int s_tot[3];
  // Per expert, the chunk counts are read 16 at a time (all loads of a batch in flight
  // together, then the in-place prefix), not one dependent round trip per chunk.
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int run = 0;
    for (int c0 = 0; c0 < nch; c0 += 16) {
      int n[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        n[u] = c0 + u < nch ? chunk_counts[(size_t)(c0 + u) * E + e] : 0;
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (c0 + u < nch) {
          chunk_counts[(size_t)(c0 + u) * E + e] = run;
          run += n[u];
        }
    }
    tot[e] = run;
    counts[e] = run;
  }
  mx_lds_sync();
  mx_dispatch_scan(tot, off, gid, mtb, s_tot, E, m_blk);
  mx_lds_sync();
  mx_dispatch_tail(tot, off, gid, mtb, s_tot, T, k, E, has_shared, m_blk, shw, offsets,
                   sorted_tok, sorted_w, g_expert, g_start, g_count, n_groups, mt_group, mt_row0,
                   n_mtiles);
}

__global__ __launch_bounds__(256) void k_dispatch_place(
    const int* __restrict__ ids, const float* __restrict__ tw, int T, int k, int E,
    const int* __restrict__ chunk_base, const int* __restrict__ rank,
    const int* __restrict__ offsets, int* __restrict__ sorted_tok, float* __restrict__ sorted_w,
    int* __restrict__ pair_pos) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= T * k) return;
  const int t = p / k;
  const int e = ids[p];
  if ((unsigned)e >= (unsigned)E) {
    pair_pos[p] = -1;
    return;
  }
  const int pos = offsets[e] + chunk_base[(size_t)(t / DC_TOK) * E + e] + rank[p];
  sorted_tok[pos] = t;
  sorted_w[pos] = tw[p];
  pair_pos[p] = pos;
}

extern "C" int mx_dispatch_scratch_size(int32_t tokens, int32_t top_k, int32_t n_experts,
                                        size_t* nbytes) {
  if (!nbytes || tokens < 0 || top_k < 1 || n_experts < 1) return MX_ERR_INVALID;
  const size_t nch = (size_t)(tokens + DC_TOK - 1) / DC_TOK;
  *nbytes = mx_align_up(nch * n_experts * 4, 256) + (size_t)tokens * top_k * 4;
  return MX_OK;
}

extern "C" int mx_dispatch_chunked(const int32_t* topk_ids, const float* topk_w,
                                   const float* shared_w, int32_t tokens, int32_t top_k,
                                   int32_t n_experts, int32_t has_shared, int32_t m_blk,
                                   void* scratch, int32_t* counts, int32_t* offsets,
                                   int32_t* sorted_tok, float* sorted_w, int32_t* pair_pos,
                                   int32_t* g_expert, int32_t* g_start, int32_t* g_count,
                                   int32_t* n_groups, int32_t* mt_group, int32_t* mt_row0,
                                   int32_t* n_mtiles, void* stream) {
  if (!topk_ids || !topk_w || !scratch || !counts || !offsets || !sorted_tok || !sorted_w ||
      !pair_pos || !g_expert || !g_start || !g_count || !n_groups || !mt_group || !mt_row0 ||
      !n_mtiles)
    return MX_ERR_INVALID;
  if (tokens < 0 || top_k < 1 || n_experts < 1 || m_blk < 1) return MX_ERR_INVALID;
  if (n_experts > 2048 || top_k > MX_DISPATCH_MAXK) return MX_ERR_UNSUPPORTED;
  if ((long)tokens * top_k > (1l << 30)) return MX_ERR_UNSUPPORTED;
  if ((size_t)n_experts * 48 > 64 * 1024) return MX_ERR_UNSUPPORTED;  // count-kernel LDS
  if (tokens == 0) return MX_OK;
  const int nch = (tokens + DC_TOK - 1) / DC_TOK;
  int* chunk = (int*)scratch;
  int* rank = (int*)((char*)scratch + mx_align_up((size_t)nch * n_experts * 4, 256));
  hipStream_t s = (hipStream_t)stream;
  mx_clear_error();
  hipLaunchKernelGGL(k_dispatch_count, dim3(nch), dim3(256), (size_t)n_experts * 48, s, topk_ids,
                     (int)tokens, (int)top_k, (int)n_experts, chunk, rank);
  MX_TRY(mx_launch_status());
  hipLaunchKernelGGL(k_dispatch_scan, dim3(1), dim3(1024), (size_t)n_experts * 16, s, shared_w,
                     (int)tokens, (int)top_k, (int)n_experts, nch, (int)has_shared, (int)m_blk,
                     chunk, counts, offsets, sorted_tok, sorted_w, g_expert, g_start, g_count,
                     n_groups, mt_group, mt_row0, n_mtiles);
  MX_TRY(mx_launch_status());
  const long pairs = (long)tokens * top_k;
  hipLaunchKernelGGL(k_dispatch_place, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s,
                     topk_ids, topk_w, (int)tokens, (int)top_k, (int)n_experts, chunk, rank,
                     offsets, sorted_tok, sorted_w, pair_pos);
  return mx_launch_status();
}
