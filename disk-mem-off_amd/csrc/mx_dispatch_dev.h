// Device body of the token -> expert dispatch, shared by k_dispatch and the fused router.
#pragma once

#include "mx_common.h"

// Largest top_k the dispatch kernels take (the router's limit as well).
#define MX_DISPATCH_MAXK 32

__host__ __device__ static inline size_t mx_dispatch_small_lds_bytes(int E) {
  return (size_t)E * 24;
}

__host__ __device__ static inline size_t mx_dispatch_lds_bytes(int nw, int E) {
  return (size_t)nw * E * 12 + (size_t)E * 16;
}

// Ordering of LDS traffic only.  A plain workgroup fence also waits for every
// outstanding global store (vmcnt(0)); these kernels communicate between threads through
// LDS alone, so their fences name the local address space and wait on lgkmcnt only.
__device__ __forceinline__ void mx_lds_fence() {  // within one wave
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ void mx_lds_sync() {  // across the workgroup
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Three exclusive scans over experts by wave 0 of the block: rows (off), active flags
// (gid) and m-tiles (mtb); totals into s_tot.  Callers synchronise (LDS) before and after.
__device__ __forceinline__ void mx_dispatch_scan(const int* tot, int* off, int* gid, int* mtb,
                                                 int* s_tot, int E, int m_blk) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // Three exclusive scans over experts by wave 0: rows, active flags, m-tiles.
  if (w == 0) {
    const int per = (E + 63) / 64;
    const int beg = min(E, lane * per), end = min(E, beg + per);
    int a = 0, b = 0, c = 0;
    for (int e = beg; e < end; ++e) {
      const int n = tot[e];
      a += n;
      b += n > 0;
      c += (n + m_blk - 1) / m_blk;
    }
    int ia = a, ib = b, ic = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int xa = __shfl_up(ia, d, 64), xb = __shfl_up(ib, d, 64), xc = __shfl_up(ic, d, 64);
      if (lane >= d) {
        ia += xa;
        ib += xb;
        ic += xc;
      }
    }
    int ea = ia - a, eb = ib - b, ec = ic - c;
    for (int e = beg; e < end; ++e) {
      const int n = tot[e];
      off[e] = ea;
      gid[e] = eb;
      mtb[e] = ec;
      ea += n;
      eb += n > 0;
      ec += (n + m_blk - 1) / m_blk;
    }
    if (lane == 63) {
      s_tot[0] = ia;
      s_tot[1] = ib;
      s_tot[2] = ic;
    }
  }
}

// Offsets, group table, m-tile list and the shared-expert rows, from the scanned tables.
__device__ __forceinline__ void mx_dispatch_tail(
    const int* tot, const int* off, const int* gid, const int* mtb, const int* s_tot, int T,
    int k, int E, int has_shared, int m_blk, const float* __restrict__ shw,
    int* __restrict__ offsets, int* __restrict__ sorted_tok, float* __restrict__ sorted_w,
    int* __restrict__ g_expert, int* __restrict__ g_start, int* __restrict__ g_count,
    int* __restrict__ n_groups, int* __restrict__ mt_group, int* __restrict__ mt_row0,
    int* __restrict__ n_mtiles) {
  const int tid = threadIdx.x;
  const int P = T * k;
  for (int e = tid; e < E; e += blockDim.x) offsets[e] = off[e];
  if (tid == 0) offsets[E] = s_tot[0];
  // Group table and m-tile list.
  const int G0 = has_shared ? 1 : 0;
  const int S0 = has_shared ? (T + m_blk - 1) / m_blk : 0;
  for (int e = tid; e < E; e += blockDim.x) {
    const int n = tot[e];
    if (n > 0) {
      const int g = G0 + gid[e];
      g_expert[g] = e;
      g_start[g] = off[e];
      g_count[g] = n;
      const int nt = (n + m_blk - 1) / m_blk;
      for (int i = 0; i < nt; ++i) {
        mt_group[S0 + mtb[e] + i] = g;
        mt_row0[S0 + mtb[e] + i] = i * m_blk;
      }
    }
  }
  if (has_shared) {
    if (tid == 0) {
      g_expert[0] = E;
      g_start[0] = P;
      g_count[0] = T;
    }
    for (int i = tid; i < S0; i += blockDim.x) {
      mt_group[i] = 0;
      mt_row0[i] = i * m_blk;
    }
    for (int t = tid; t < T; t += blockDim.x) {
      sorted_tok[P + t] = t;
      sorted_w[P + t] = shw ? shw[t] : 1.f;
    }
  }
  if (tid == 0) {
    *n_groups = G0 + s_tot[1];
    *n_mtiles = S0 + s_tot[2];
  }
}

// Whole-workgroup dispatch (every thread of the block must call it).  `smem` holds
// mx_dispatch_lds_bytes(blockDim.x / 64, E) bytes.
__device__ __forceinline__ void mx_dispatch_block(
    unsigned char* smem, const int* __restrict__ ids, const float* __restrict__ tw,
    const float* __restrict__ shw, int T, int k, int E, int has_shared, int m_blk,
    int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ sorted_tok,
    float* __restrict__ sorted_w, int* __restrict__ pair_pos, int* __restrict__ g_expert,
    int* __restrict__ g_start, int* __restrict__ g_count, int* __restrict__ n_groups,
    int* __restrict__ mt_group, int* __restrict__ mt_row0, int* __restrict__ n_mtiles) {
  const int NW = blockDim.x >> 6;
  unsigned long long* mask = (unsigned long long*)smem;  // [NW][E]
  int* cnt = (int*)(mask + (size_t)NW * E);             // [NW][E]
  int* tot = cnt + NW * E;                               // [E]
  int* off = tot + E;                                    // [E]
  int* gid = off + E;                                    // [E]
  int* mtb = gid + E;                                    // [E]
  __shared__ int s_tot[3];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int P = T * k;
  const int tpw = (T + NW - 1) / NW;
  const int tb = min(T, w * tpw), te = min(T, tb + tpw);

  for (int i = tid; i < NW * E; i += blockDim.x) cnt[i] = 0;
  mx_lds_sync();
  for (int p = tb * k + lane; p < te * k; p += 64) {
    const int e = ids[p];
    if ((unsigned)e < (unsigned)E) atomicAdd(&cnt[w * E + e], 1);
  }
  mx_lds_sync();
  // Per expert: exclusive base of every wave's range, and the total.
  for (int e = tid; e < E; e += blockDim.x) {
    int run = 0;
    for (int ww = 0; ww < NW; ++ww) {
      const int c = cnt[ww * E + e];
      cnt[ww * E + e] = run;
      run += c;
    }
    tot[e] = run;
    counts[e] = run;
  }
  mx_lds_sync();
  mx_dispatch_scan(tot, off, gid, mtb, s_tot, E, m_blk);
  mx_lds_sync();

  // Stable positions: rounds of 64 tokens per wave, lane = token.  Mask reads follow an
  // LDS fence and go through the LDS pointer (a volatile access would drop the address
  // space and become a system-coherent flat load).
  unsigned long long* wm = mask + (size_t)w * E;
  int* wc = cnt + w * E;
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int r0 = tb; r0 < te; r0 += 64) {
    const int t = r0 + lane;
    const bool v = t < te;
    for (int j = 0; j < k; ++j) {
      const int e = v ? ids[t * k + j] : -1;
      if ((unsigned)e < (unsigned)E) wm[e] = 0ull;
    }
    mx_lds_fence();
    for (int j = 0; j < k; ++j) {
      const int e = v ? ids[t * k + j] : -1;
      if ((unsigned)e < (unsigned)E) atomicOr(&wm[e], 1ull << lane);
    }
    mx_lds_fence();
    for (int j = 0; j < k; ++j) {
      if (!v) break;
      const int e = ids[t * k + j];
      if ((unsigned)e < (unsigned)E) {
        const int pos = off[e] + wc[e] + __popcll(wm[e] & below);
        sorted_tok[pos] = t;
        sorted_w[pos] = tw[t * k + j];
        pair_pos[t * k + j] = pos;
      } else {
        pair_pos[t * k + j] = -1;
      }
    }
    if (r0 + 64 < te) {  // another round of this wave's range follows
      mx_lds_fence();
      for (int j = 0; j < k; ++j) {
        const int e = v ? ids[t * k + j] : -1;
        if ((unsigned)e < (unsigned)E) {
          const unsigned long long m = wm[e];
          if ((m & below) == 0ull) wc[e] += __popcll(m);
        }
      }
      mx_lds_fence();
    }
  }
  mx_lds_sync();
  mx_dispatch_tail(tot, off, gid, mtb, s_tot, T, k, E, has_shared, m_blk, shw, offsets,
                   sorted_tok, sorted_w, g_expert, g_start, g_count, n_groups, mt_group, mt_row0,
                   n_mtiles);
}


// Dispatch of at most 64 tokens (decode batches), whole workgroup.  Token t is bit t of
// a per-expert 64-bit mask: mask[e] = tokens that chose e, count = popcount, and the
// row of pair (t, j) inside expert e = popcount of the mask bits below t, i.e. ascending
// token order with no per-wave ranges or rounds.  `smem` holds
// mx_dispatch_small_lds_bytes(E) bytes; ids / tw / shw may point to LDS.
__device__ __forceinline__ void mx_dispatch_block_small(
    unsigned char* smem, const int* ids, const float* tw, const float* shw, int T, int k,
    int E, int has_shared, int m_blk, int* __restrict__ counts, int* __restrict__ offsets,
    int* __restrict__ sorted_tok, float* __restrict__ sorted_w, int* __restrict__ pair_pos,
    int* __restrict__ g_expert, int* __restrict__ g_start, int* __restrict__ g_count,
    int* __restrict__ n_groups, int* __restrict__ mt_group, int* __restrict__ mt_row0,
    int* __restrict__ n_mtiles) {
  unsigned long long* mask = (unsigned long long*)smem;  // [E]
  int* tot = (int*)(mask + E);                          // [E]
  int* off = tot + E;                                    // [E]
  int* gid = off + E;                                    // [E]
  int* mtb = gid + E;                                    // [E]
  __shared__ int s_tot[3];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int P = T * k;
  for (int e = tid; e < E; e += nt) mask[e] = 0ull;
  mx_lds_sync();
  for (int p = tid; p < P; p += nt) {
    const int e = ids[p];
    if ((unsigned)e < (unsigned)E) atomicOr(&mask[e], 1ull << (p / k));
  }
  mx_lds_sync();
  for (int e = tid; e < E; e += nt) {
    const int n = __popcll(mask[e]);
    tot[e] = n;
    counts[e] = n;
  }
  mx_lds_sync();
  mx_dispatch_scan(tot, off, gid, mtb, s_tot, E, m_blk);
  mx_lds_sync();
  for (int p = tid; p < P; p += nt) {
    const int e = ids[p], t = p / k;
    if ((unsigned)e < (unsigned)E) {
      const int pos = off[e] + __popcll(mask[e] & ((1ull << t) - 1ull));
      sorted_tok[pos] = t;
      sorted_w[pos] = tw[p];
      pair_pos[p] = pos;
    } else {
      pair_pos[p] = -1;
    }
  }
  mx_dispatch_tail(tot, off, gid, mtb, s_tot, T, k, E, has_shared, m_blk, shw, offsets,
                   sorted_tok, sorted_w, g_expert, g_start, g_count, n_groups, mt_group, mt_row0,
                   n_mtiles);
}
