// Device-side building blocks shared by the standalone and the fused router kernels.
#pragma once

#include <math.h>

#include "mx_common.h"

#define TK_MAXK 32

// One wave selects the experts of token t (logits summed over S H-slices).
template <int VPT>
__device__ __forceinline__ void mx_topk_token(
    const float* __restrict__ logits, int S, int T, int t, const void* __restrict__ bias,
    int pdt, int E, int E1, int k, int mode, int norm, float scaling, int has_seg,
    int* __restrict__ ids, float* __restrict__ tw, float* __restrict__ shared_w,
    int* lds_ids = nullptr, float* lds_w = nullptr, float* lds_sw = nullptr) {
  const int lane = threadIdx.x & 63;
  float key[VPT], wsrc[VPT];
  bool taken[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = lane + 64 * i;
    taken[i] = false;
    key[i] = -INFINITY;
    wsrc[i] = 0.f;
    if (e < E) {
      float l = 0.f;
      for (int s = 0; s < S; ++s) l += logits[((size_t)s * T + t) * E1 + e];
      const float b = bias ? mx_load_param(bias, pdt, e) : 0.f;
      if (mode == MX_ROUTER_SIGMOID_SELECT_BIAS) {
        const float sg = mx_sigmoid(l);
        key[i] = sg + b;
        wsrc[i] = sg;
      } else {
        key[i] = (mode == MX_ROUTER_REF_SOFTMAX_BIAS) ? l + b : l;
      }
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
#pragma unroll
  for (int i = 0; i < VPT; ++i)
    if (key[i] != key[i]) key[i] = -INFINITY;  // NaN never wins a slot

  // Lane r keeps selection r (no dynamically indexed private arrays).
  int my_id = 0;
  float my_w = 0.f;
  for (int r = 0; r < k; ++r) {
    float bk = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !taken[i] && (key[i] > bk || (key[i] == bk && e < bi))) {
        bk = key[i];
        bi = e;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ok = __shfl_xor(bk, m, 64);
      const int oi = __shfl_xor(bi, m, 64);
      if (ok > bk || (ok == bk && oi < bi)) {
        bk = ok;
        bi = oi;
      }
    }
    const int wl = bi & 63, wi = bi >> 6;
    float mine = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      if (i == wi) {
        mine = wsrc[i];
        if (lane == wl) taken[i] = true;
      }
    }
    const float w = __shfl(mine, wl, 64);
    if (lane == r) {
      my_id = bi;
      my_w = w;
    }
  }
  float sum = 0.f;  // sequential over the k slots, identical on every lane
  for (int r = 0; r < k; ++r) sum += __shfl(my_w, r, 64);
  if (lane < k) {
    const float w = (norm ? my_w / (sum + 1e-20f) : my_w) * scaling;
    ids[(size_t)t * k + lane] = my_id;
    tw[(size_t)t * k + lane] = w;
    if (lds_ids) {
      lds_ids[t * k + lane] = my_id;
      lds_w[t * k + lane] = w;
    }
  }
  if (lane == 0) {
    if (shared_w) {
      float g = 1.f;
      if (has_seg) {
        float l = 0.f;
        for (int s = 0; s < S; ++s) l += logits[((size_t)s * T + t) * E1 + E];
        g = mx_sigmoid(l);
      }
      shared_w[t] = g;
      if (lds_sw) lds_sw[t] = g;
    }
  }
}


#include "mx_dispatch_dev.h"
