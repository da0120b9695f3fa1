// Device-side building blocks shared by the standalone and the fused router kernels.
#pragma once

#include <math.h>

#include "mx_common.h"
#include "mx_dispatch_dev.h"

#define TK_MAXK 32

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
  for (int s = 1; s < S; ++s)
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      lg[i] += logits[((size_t)s * T + t) * E1 + min(lane + 64 * i, E - 1)];
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

  // Selection without a per-round arg-max.  Keys map to order-preserving 32-bit images
  // (NaN counts as -inf, -0 as +0; 0 marks an absent expert).  A most-significant-bit-first
  // search with wave ballots finds tau, the k-th largest image; every image above tau is
  // taken, and the ties at tau in ascending expert id until k are filled.  A chosen
  // expert's slot is the number of chosen experts ahead of it (larger key, or equal key
  // and lower id), i.e. the order k rounds of arg-max with ties to the lower id give.
  uint32_t u[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    float kv = key[i];
    if (kv != kv) kv = -INFINITY;
    if (kv == 0.f) kv = 0.f;
    const uint32_t b = __builtin_bit_cast(uint32_t, kv);
    u[i] = (lane + 64 * i < E) ? ((b & 0x80000000u) ? ~b : (b | 0x80000000u)) : 0u;
  }
  uint32_t tau = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = tau | (1u << bit);
    unsigned long long m[VPT];  // all compares first: independent mask registers
#pragma unroll
    for (int i = 0; i < VPT; ++i) m[i] = __builtin_amdgcn_uicmp(u[i], cand, 35 /* uge */);
    int c = 0;
#pragma unroll
    for (int i = 0; i < VPT; ++i) c += __popcll(m[i]);
    if (c >= k) tau = cand;
  }
  const unsigned long long below = (1ull << lane) - 1ull;
  int ngt = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) ngt += __popcll(__ballot(u[i] > tau));
  bool sel[VPT];
  int ties = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const unsigned long long eq = __ballot(u[i] == tau);
    sel[i] = u[i] > tau || (u[i] == tau && ties + __popcll(eq & below) < k - ngt);
    ties += __popcll(eq);
  }
  int rank[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) rank[i] = 0;
#pragma unroll
  for (int iy = 0; iy < VPT; ++iy) {
    unsigned long long m = __ballot(sel[iy]);
    while (m) {
      const int ly = __builtin_ctzll(m);
      m &= m - 1ull;
      const uint32_t uy = (uint32_t)__builtin_amdgcn_readlane((int)u[iy], ly);
      const int ey = ly + 64 * iy;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        rank[i] += (uy > u[i] || (uy == u[i] && ey < lane + 64 * i)) ? 1 : 0;
    }
  }
  // Chosen experts land in their slots of a per-wave LDS row; lane r then owns slot r.
  __shared__ int s_id[16][TK_MAXK];
  __shared__ float s_w[16][TK_MAXK];
  const int wv = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    if (sel[i]) {
      s_id[wv][rank[i]] = lane + 64 * i;
      s_w[wv][rank[i]] = wsrc[i];
    }
  }
  mx_lds_fence();
  const int my_id = lane < k ? s_id[wv][lane] : 0;
  const float my_w = lane < k ? s_w[wv][lane] : 0.f;
  mx_lds_fence();  // the row is reused by this wave's next token
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

__device__ __forceinline__ uint32_t mx_key_image(float kv, bool valid) {
  if (kv != kv) kv = -INFINITY;
  if (kv == 0.f) kv = 0.f;
  const uint32_t b = __builtin_bit_cast(uint32_t, kv);
  return valid ? ((b & 0x80000000u) ? ~b : (b | 0x80000000u)) : 0u;
}

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
  uint32_t tau = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = tau | (1u << bit);
    int c = 0;
#pragma unroll
    for (int i = 0; i < VPC; ++i) c += __popcll(__builtin_amdgcn_uicmp(u[i], cand, 35 /* uge */));
    if (c >= k) tau = cand;
  }
  const unsigned long long below = (1ull << lane) - 1ull;
  int ngt = 0;
#pragma unroll
  for (int i = 0; i < VPC; ++i) ngt += __popcll(__ballot(u[i] > tau));
  int ties = 0, ahead = 0;
#pragma unroll
  for (int i = 0; i < VPC; ++i) {
    const unsigned long long eq = __ballot(u[i] == tau);
    const bool sel = u[i] > tau || (u[i] == tau && ties + __popcll(eq & below) < k - ngt);
    ties += __popcll(eq);
    const unsigned long long sm = __ballot(sel);
    if (sel) {
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
  uint32_t tau = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = tau | (1u << bit);
    int c = 0;
#pragma unroll
    for (int i = 0; i < VC; ++i) c += __popcll(__builtin_amdgcn_uicmp(u[i], cand, 35));
    if (c >= k) tau = cand;
  }
  const unsigned long long below = (1ull << lane) - 1ull;
  int ngt = 0;
#pragma unroll
  for (int i = 0; i < VC; ++i) ngt += __popcll(__ballot(u[i] > tau));
  bool sel[VC];
  int ties = 0;
#pragma unroll
  for (int i = 0; i < VC; ++i) {
    const unsigned long long eq = __ballot(u[i] == tau);
    sel[i] = u[i] > tau || (u[i] == tau && ties + __popcll(eq & below) < k - ngt);
    ties += __popcll(eq);
  }
  // Slot = number of chosen candidates ahead (larger image, or equal and lower id).
  int rank[VC];
#pragma unroll
  for (int i = 0; i < VC; ++i) rank[i] = 0;
#pragma unroll
  for (int iy = 0; iy < VC; ++iy) {
    unsigned long long m = __ballot(sel[iy]);
    while (m) {
      const int ly = __builtin_ctzll(m);
      m &= m - 1ull;
      const uint32_t uy = (uint32_t)__builtin_amdgcn_readlane((int)u[iy], ly);
      const int ey = __builtin_amdgcn_readlane(cid[iy], ly);
#pragma unroll
      for (int i = 0; i < VC; ++i) rank[i] += (uy > u[i] || (uy == u[i] && ey < cid[i])) ? 1 : 0;
    }
  }
  float M = 0.f, S = 1.f;
  if (mode != MX_ROUTER_SIGMOID_SELECT_BIAS) {
    M = -INFINITY;
    for (int p = 0; p < NP; ++p) M = fmaxf(M, sh.m[t * NP + p]);
    S = 0.f;
    for (int p = 0; p < NP; ++p) S += sh.sm[t * NP + p] * expf(sh.m[t * NP + p] - M);
  }
  __shared__ int s_id[16][TK_MAXK];
  __shared__ float s_w[16][TK_MAXK];
  const int wv = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < VC; ++i) {
    if (sel[i]) {
      s_id[wv][rank[i]] = cid[i];
      s_w[wv][rank[i]] =
          mode == MX_ROUTER_SIGMOID_SELECT_BIAS ? cw[i] : expf(cw[i] - M) / S;
    }
  }
  mx_lds_fence();
  const int my_id = lane < k ? s_id[wv][lane] : 0;
  const float my_w = lane < k ? s_w[wv][lane] : 0.f;
  mx_lds_fence();  // the row is reused by this wave's next call
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
