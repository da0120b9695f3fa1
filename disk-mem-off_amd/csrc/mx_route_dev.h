// Device-side building blocks shared by the standalone and the fused router kernels.
#pragma once

#include <math.h>

#include "mx_common.h"
#include "mx_dispatch_dev.h"

#define TK_MAXK 32
#ifndef TK_SB
#define TK_SB 4  // logit slices loaded together by the top-k
#endif

// ---- selection core shared by the top-k variants ----------------------------------
// Images: keys mapped to order-preserving 32-bit values (NaN counts as -inf, -0 as +0;
// 0 marks an absent entry).  A most-significant-bit-first search with wave ballots finds
// a threshold tau with exactly the k largest images at or above it when they are distinct
// from the rest: the search stops as soon as the count at the candidate is exactly k
// (random keys: after about log2(entries) + 3 of the 32 steps); otherwise it ends at the
// k-th largest image.  Every image above tau is chosen, and the ties at tau in ascending
// entry order until k are filled, so the chosen set is the one k rounds of arg-max with
// ties to the lower entry give.
__device__ __forceinline__ uint32_t mx_key_image(float kv, bool valid) {
  if (kv != kv) kv = -INFINITY;
  if (kv == 0.f) kv = 0.f;
  const uint32_t b = __builtin_bit_cast(uint32_t, kv);
  return valid ? ((b & 0x80000000u) ? ~b : (b | 0x80000000u)) : 0u;
}

template <int V>
__device__ __forceinline__ void mx_choose_k(const uint32_t (&u)[V], int k, bool (&sel)[V]) {
  const int lane = threadIdx.x & 63;
  uint32_t tau = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = tau | (1u << bit);
    unsigned long long m[V];  // all compares first: independent mask registers
#pragma unroll
    for (int i = 0; i < V; ++i) m[i] = __builtin_amdgcn_uicmp(u[i], cand, 35 /* uge */);
    int c = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) c += __popcll(m[i]);
    if (c >= k) {
      tau = cand;
      if (c == k) break;
    }
  }
  const unsigned long long below = (1ull << lane) - 1ull;
  int ngt = 0;
#pragma unroll
  for (int i = 0; i < V; ++i) ngt += __popcll(__ballot(u[i] > tau));
  int ties = 0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const unsigned long long eq = __ballot(u[i] == tau);
    sel[i] = u[i] > tau || (u[i] == tau && ties + __popcll(eq & below) < k - ngt);
    ties += __popcll(eq);
  }
}

// Slots of the k chosen entries (image, id, payload): slot = number of chosen entries
// ahead (larger image, or equal image and lower id).  The chosen are packed into a
// per-wave LDS row in entry order, lane r < k takes entry r and counts the entries
// ahead of it with k wave-uniform reads, and the packed row is rewritten in slot order;
// lane r < k returns slot r's id and payload.
template <int V>
__device__ __forceinline__ void mx_slots_of(const bool (&sel)[V], const uint32_t (&u)[V],
                                            const int (&id)[V], const float (&w)[V], int k,
                                            int& my_id, float& my_w) {
  __shared__ uint32_t s_u[16][TK_MAXK];
  __shared__ int s_id[16][TK_MAXK];
  __shared__ float s_w[16][TK_MAXK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const unsigned long long below = (1ull << lane) - 1ull;
  int ahead = 0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const unsigned long long m = __ballot(sel[i]);
    if (sel[i]) {
      const int pos = ahead + __popcll(m & below);
      s_u[wv][pos] = u[i];
      s_id[wv][pos] = id[i];
      s_w[wv][pos] = w[i];
    }
    ahead += __popcll(m);
  }
  mx_lds_fence();
  const uint32_t ur = lane < k ? s_u[wv][lane] : 0u;
  const int ir = lane < k ? s_id[wv][lane] : 0;
  const float wr = lane < k ? s_w[wv][lane] : 0.f;
  mx_lds_fence();  // every lane has its entry before the row is rewritten
  int rank = 0;
  for (int j = 0; j < k; ++j) {
    const uint32_t uj = (uint32_t)__builtin_amdgcn_readlane((int)ur, j);
    const int ij = __builtin_amdgcn_readlane(ir, j);
    rank += (uj > ur || (uj == ur && ij < ir)) ? 1 : 0;
  }
  if (lane < k) {
    s_id[wv][rank] = ir;
    s_w[wv][rank] = wr;
  }
  mx_lds_fence();
  my_id = lane < k ? s_id[wv][lane] : 0;
  my_w = lane < k ? s_w[wv][lane] : 0.f;
  mx_lds_fence();  // the rows are reused by this wave's next call
}

// The selection of one token by one wave: lane r < k holds slot r's expert id and its
// final weight (renormalised and scaled as configured).
struct MxSel {
  int id;
  float w;
};

// One wave selects the experts of token t (logits summed over S H-slices).
template <int VPT>
__device__ __forceinline__ MxSel mx_topk_select(const float* __restrict__ logits, int S, int T,
                                                int t, const void* __restrict__ bias, int pdt,
                                                int E, int E1, int k, int mode, int norm,
                                                float scaling) {
  const int lane = threadIdx.x & 63;
  // All logit and bias loads first, at clamped indices, so they are in flight together.
  float lg[VPT], bs[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    lg[i] = logits[(size_t)t * E1 + min(lane + 64 * i, E - 1)];
    bs[i] = 0.f;
  }
  if (bias && pdt == MX_DT_F16) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) bs[i] = (float)((const half_t*)bias)[min(lane + 64 * i, E - 1)];
  } else if (bias) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) bs[i] = ((const float*)bias)[min(lane + 64 * i, E - 1)];
  }
  // Later slices TK_SB at a time: every load of a batch is issued (slice index clamped)
  // before the adds, which run in slice order and skip the clamped repeats.
  for (int s0 = 1; s0 < S; s0 += TK_SB) {
    float ps[TK_SB][VPT];
#pragma unroll
    for (int u = 0; u < TK_SB; ++u)
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        ps[u][i] = logits[((size_t)min(s0 + u, S - 1) * T + t) * E1 + min(lane + 64 * i, E - 1)];
#pragma unroll
    for (int u = 0; u < TK_SB; ++u)
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        if (s0 + u < S) lg[i] += ps[u][i];
  }
  float key[VPT], wsrc[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const bool valid = lane + 64 * i < E;
    const float l = lg[i];
    if (mode == MX_ROUTER_SIGMOID_SELECT_BIAS) {
      const float sg = mx_sigmoid(l);
      key[i] = valid ? sg + bs[i] : -INFINITY;
      wsrc[i] = valid ? sg : 0.f;
    } else {
      key[i] = valid ? ((mode == MX_ROUTER_REF_SOFTMAX_BIAS) ? l + bs[i] : l) : -INFINITY;
      wsrc[i] = 0.f;
    }
  }
  if (mode != MX_ROUTER_SIGMOID_SELECT_BIAS) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) m = fmaxf(m, key[i]);
    m = mx_wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = lane + 64 * i;
      wsrc[i] = (e < E) ? expf(key[i] - m) : 0.f;
      sum += wsrc[i];
    }
    sum = mx_wave_sum(sum);
#pragma unroll
    for (int i = 0; i < VPT; ++i) wsrc[i] = wsrc[i] / sum;
  }

  uint32_t u[VPT];
  int eid[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    eid[i] = lane + 64 * i;
    u[i] = mx_key_image(key[i], eid[i] < E);
  }
  bool sel[VPT];
  mx_choose_k(u, k, sel);
  int my_id;
  float my_w;
  mx_slots_of(sel, u, eid, wsrc, k, my_id, my_w);
  float sum = 0.f;  // sequential over the k slots, identical on every lane
  for (int r = 0; r < k; ++r) sum += mx_readlane(my_w, r);
  return MxSel{my_id, (norm ? my_w / (sum + 1e-20f) : my_w) * scaling};
}

// Weight of the shared expert's row: sigmoid of the shared-gate logit (Qwen3-Next), else 1.
__device__ __forceinline__ float mx_shared_gate(const float* __restrict__ logits, int S, int T,
                                                int t, int E, int E1, int has_seg) {
  float g = 1.f;
  if (has_seg) {
    float l = 0.f;
    for (int s = 0; s < S; ++s) l += logits[((size_t)s * T + t) * E1 + E];
    g = mx_sigmoid(l);
  }
  return g;
}

// One wave selects token t and writes its ids / weights (and the shared weight).
template <int VPT>
__device__ __forceinline__ void mx_topk_token(
    const float* __restrict__ logits, int S, int T, int t, const void* __restrict__ bias,
    int pdt, int E, int E1, int k, int mode, int norm, float scaling, int has_seg,
    int* __restrict__ ids, float* __restrict__ tw, float* __restrict__ shared_w,
    int* lds_ids = nullptr, float* lds_w = nullptr, float* lds_sw = nullptr) {
  const int lane = threadIdx.x & 63;
  const MxSel sel = mx_topk_select<VPT>(logits, S, T, t, bias, pdt, E, E1, k, mode, norm, scaling);
  if (lane < k) {
    ids[(size_t)t * k + lane] = sel.id;
    tw[(size_t)t * k + lane] = sel.w;
    if (lds_ids) {
      lds_ids[t * k + lane] = sel.id;
      lds_w[t * k + lane] = sel.w;
    }
  }
  if (lane == 0 && shared_w) {
    const float g = mx_shared_gate(logits, S, T, t, E, E1, has_seg);
    shared_w[t] = g;
    if (lds_sw) lds_sw[t] = g;
  }
}

// Dispatch tables of a one-token batch, written by the wave that selected it (lane r < k
// holds slot r's id and weight): every chosen expert is a group of one row, groups in
// ascending expert id (the order of the general dispatch), the shared expert's row last
// and its group and tile first.
__device__ __forceinline__ void mx_dispatch_one_token(
    int my_id, float my_w, float shared_gate, int k, int E, int has_shared,
    int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ sorted_tok,
    float* __restrict__ sorted_w, int* __restrict__ pair_pos, int* __restrict__ g_expert,
    int* __restrict__ g_start, int* __restrict__ g_count, int* __restrict__ n_groups,
    int* __restrict__ mt_group, int* __restrict__ mt_row0, int* __restrict__ n_mtiles) {
  const int lane = threadIdx.x & 63;
  const int G0 = has_shared ? 1 : 0, S0 = has_shared ? 1 : 0;
  const int id = lane < k ? my_id : 0x7fffffff;
  int rank = 0;
  for (int i = 0; i < k; ++i) rank += __builtin_amdgcn_readlane(id, i) < id ? 1 : 0;
  if (lane < k) {
    sorted_tok[rank] = 0;
    sorted_w[rank] = my_w;
    pair_pos[lane] = rank;
    g_expert[G0 + rank] = id;
    g_start[G0 + rank] = rank;
    g_count[G0 + rank] = 1;
    mt_group[S0 + rank] = G0 + rank;
    mt_row0[S0 + rank] = 0;
  }
  for (int e = lane; e <= E; e += 64) {
    int below = 0, hit = 0;
    for (int i = 0; i < k; ++i) {
      const int x = __builtin_amdgcn_readlane(id, i);
      below += x < e ? 1 : 0;
      hit |= x == e ? 1 : 0;
    }
    if (e < E) counts[e] = hit;
    offsets[e] = below;
  }
  if (lane == 0) {
    if (has_shared) {
      g_expert[0] = E;
      g_start[0] = k;
      g_count[0] = 1;
      mt_group[0] = 0;
      mt_row0[0] = 0;
      sorted_tok[k] = 0;
      sorted_w[k] = shared_gate;
    }
    *n_groups = G0 + k;
    *n_mtiles = S0 + k;
  }
}

// ------------------------------------------------------------------------------------
// Top-k of small batches spread over several waves per token (the same selection and
// weights as mx_topk_token).  Token t takes NP = ceil(E / 64) waves; wave `part` holds
// experts 64 part .. 64 part + 63, one per lane, and keeps its k largest (key image,
// then lower id) as candidates in LDS, in ascending expert id.  Every expert of the
// token's top-k is among its wave's k, so one wave per token then selects the top-k of
// the NP k candidates; the candidate order is the expert id order, which keeps the tie
// rule.  Softmax weights use the per-wave maxima and sums: M = max_p m_p,
// S = sum_p s_p exp(m_p - M) (parts in order).
// ------------------------------------------------------------------------------------
#define TKP_MAXC 512  // candidates per block: (tokens x parts) <= 16 waves, k <= 32

struct MxTopkPar {
  uint32_t u[TKP_MAXC];
  int id[TKP_MAXC];
  float w[TKP_MAXC];  // sigmoid score (sigmoid modes) or key (softmax modes)
  float m[16], sm[16];
};


// Phase 1, by wave `wv` < T * NP of the block: candidates of token wv / NP.  A part holds
// 64 * VPC consecutive experts (VPC per lane, lane-major within each 64).
template <int VPC = 1>
__device__ __forceinline__ void mx_topk_par_cand(MxTopkPar& sh, const float* __restrict__ logits,
                                                 const void* __restrict__ bias, int pdt, int E,
                                                 int E1, int k, int mode, int NP, int wv) {
  const int lane = threadIdx.x & 63;
  const int t = wv / NP, part = wv - t * NP;
  bool valid[VPC];
  float key[VPC], wsrc[VPC];
#pragma unroll
  for (int i = 0; i < VPC; ++i) {
    const int e = part * 64 * VPC + 64 * i + lane;
    valid[i] = e < E;
    const int ec = min(e, E - 1);
    const float l = logits[(size_t)t * E1 + ec];
    float b = 0.f;
    if (bias) b = pdt == MX_DT_F16 ? (float)((const half_t*)bias)[ec] : ((const float*)bias)[ec];
    if (mode == MX_ROUTER_SIGMOID_SELECT_BIAS) {
      wsrc[i] = mx_sigmoid(l);
      key[i] = valid[i] ? wsrc[i] + b : -INFINITY;
    } else {
      key[i] = valid[i] ? ((mode == MX_ROUTER_REF_SOFTMAX_BIAS) ? l + b : l) : -INFINITY;
      wsrc[i] = key[i];
    }
  }
  if (mode != MX_ROUTER_SIGMOID_SELECT_BIAS) {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPC; ++i) mx = fmaxf(mx, key[i]);
    const float m = mx_wave_max(mx);
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < VPC; ++i) ls += valid[i] ? expf(key[i] - m) : 0.f;
    const float sm = mx_wave_sum(ls);
    if (lane == 0) {
      sh.m[wv] = m;
      sh.sm[wv] = sm;
    }
  }
  uint32_t u[VPC];
#pragma unroll
  for (int i = 0; i < VPC; ++i) u[i] = mx_key_image(key[i], valid[i]);
  bool sel[VPC];
  mx_choose_k(u, k, sel);
  const unsigned long long below = (1ull << lane) - 1ull;
  int ahead = 0;
#pragma unroll
  for (int i = 0; i < VPC; ++i) {
    const unsigned long long sm = __ballot(sel[i]);
    if (sel[i]) {
      const int slot = t * NP * k + part * k + ahead + __popcll(sm & below);
      sh.u[slot] = u[i];
      sh.id[slot] = part * 64 * VPC + 64 * i + lane;
      sh.w[slot] = wsrc[i];
    }
    ahead += __popcll(sm);
  }
}

// Phase 2, by one wave per token (after a workgroup LDS sync): the token's top-k, returned
// like mx_topk_select (lane r < k: slot r's id and final weight).
template <int VC>
__device__ __forceinline__ MxSel mx_topk_par_select(const MxTopkPar& sh, int t, int k, int mode,
                                                    int norm, float scaling, int NP) {
  const int lane = threadIdx.x & 63;
  const int C = NP * k, c0 = t * C;
  uint32_t u[VC];
  int cid[VC];
  float cw[VC];
#pragma unroll
  for (int i = 0; i < VC; ++i) {
    const int s = lane + 64 * i;
    const bool v = s < C;
    u[i] = v ? sh.u[c0 + s] : 0u;
    cid[i] = v ? sh.id[c0 + s] : 0;
    cw[i] = v ? sh.w[c0 + s] : 0.f;
  }
  bool sel[VC];
  mx_choose_k(u, k, sel);
  float M = 0.f, S = 1.f;
  if (mode != MX_ROUTER_SIGMOID_SELECT_BIAS) {
    M = -INFINITY;
    for (int p = 0; p < NP; ++p) M = fmaxf(M, sh.m[t * NP + p]);
    S = 0.f;
    for (int p = 0; p < NP; ++p) S += sh.sm[t * NP + p] * expf(sh.m[t * NP + p] - M);
  }
  int my_id;
  float my_w;
  mx_slots_of(sel, u, cid, cw, k, my_id, my_w);
  if (lane < k && mode != MX_ROUTER_SIGMOID_SELECT_BIAS) my_w = expf(my_w - M) / S;
  float sum = 0.f;  // sequential over the k slots, identical on every lane
  for (int r = 0; r < k; ++r) sum += mx_readlane(my_w, r);
  return MxSel{my_id, (norm ? my_w / (sum + 1e-20f) : my_w) * scaling};
}

// Phase 2 with the results written out (ids / weights / shared weight, global and LDS).
template <int VC>
__device__ __forceinline__ void mx_topk_par_final(
    const MxTopkPar& sh, const float* __restrict__ logits, int t, int E, int E1, int k,
    int mode, int norm, float scaling, int NP, int has_seg, int* __restrict__ ids,
    float* __restrict__ tw, float* __restrict__ shared_w, int* lds_ids, float* lds_w,
    float* lds_sw) {
  const int lane = threadIdx.x & 63;
  const MxSel sel = mx_topk_par_select<VC>(sh, t, k, mode, norm, scaling, NP);
  if (lane < k) {
    ids[(size_t)t * k + lane] = sel.id;
    tw[(size_t)t * k + lane] = sel.w;
    lds_ids[t * k + lane] = sel.id;
    lds_w[t * k + lane] = sel.w;
  }
  if (lane == 0 && shared_w) {
    const float g = has_seg ? mx_sigmoid(logits[(size_t)t * E1 + E]) : 1.f;
    shared_w[t] = g;
    lds_sw[t] = g;
  }
}
