// RMSNorm, router logits and router top-k for the MoE block.
//
// Reference: offload_runtime/executors/glm4_moe.py:177-200 (GLM4-MoE) and
// offload_runtime/executors/qwen3_next.py:274-293, :327-329 (Qwen3-Next), with the
// primitives rms_norm / softmax of offload_runtime/executors/_common.py:73-75, :87-90.
// All arithmetic is fp32, as in the NumPy reference (fp16 parameters are widened first).
#include <math.h>

#include "mx_common.h"
#include "mx_internal.h"

// ------------------------------------------------------------------------------------
// RMSNorm: one 256-thread block per token.  h = w * (x / sqrt(mean(x^2) + eps)).
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x,
                                                 const void* __restrict__ w, int wdt,
                                                 float eps, int H, float* __restrict__ h32,
                                                 half_t* __restrict__ h16) {
  const int t = blockIdx.x;
  const float* xr = x + (size_t)t * H;
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += 256) {
    float v = xr[i];
    ss = fmaf(v, v, ss);
  }
  __shared__ float red[4];
  ss = mx_wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float rms = sqrtf(ss / (float)H + eps);
  float* hr = h32 + (size_t)t * H;
  half_t* hr16 = h16 ? h16 + (size_t)t * H : nullptr;
  for (int i = threadIdx.x; i < H; i += 256) {
    float v = mx_load_param(w, wdt, i) * (xr[i] / rms);
    hr[i] = v;
    if (hr16) hr16[i] = (half_t)v;
  }
}

extern "C" int mx_rmsnorm(const float* x, const void* norm_w, int32_t param_dtype, float eps,
                          int32_t tokens, int32_t hidden, float* h32, void* h16, void* stream) {
  if (!x || !norm_w || !h32 || tokens < 0 || hidden <= 0) return MX_ERR_INVALID;
  if (param_dtype != MX_DT_F32 && param_dtype != MX_DT_F16) return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  mx_clear_error();
  hipLaunchKernelGGL(k_rmsnorm, dim3(tokens), dim3(256), 0, (hipStream_t)stream, x, norm_w,
                     (int)param_dtype, eps, (int)hidden, h32, (half_t*)h16);
  return mx_launch_status();
}

// ------------------------------------------------------------------------------------
// Router logits, split over H.  Block = 4 waves; wave w owns experts e0..e0+3 of the
// block's 16-expert tile and RT_TT tokens.  Lanes stride H by 4 elements; each wave
// reduces its RT_TT x 4 partial dot products at the end.  Row e == E is the Qwen3-Next
// shared-expert gate (qwen3_next.py:328), which rides along as an extra "expert".
// out[s][t][e] holds the partial sum of H-slice s; the top-k kernel adds the slices in
// ascending order, so the result does not depend on scheduling.
// ------------------------------------------------------------------------------------
#define RT_TT 8
#define RT_EPB 16
#define RT_KCH 256  // H elements per lane sweep (64 lanes x 4)

template <typename WT>
__device__ __forceinline__ float4 rt_load4(const WT* p);
template <>
__device__ __forceinline__ float4 rt_load4<float>(const float* p) {
  return *(const float4*)p;
}
template <>
__device__ __forceinline__ float4 rt_load4<half_t>(const half_t* p) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  h4 v = *(const h4*)p;
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

template <typename WT>
__global__ __launch_bounds__(256) void k_router_logits(const float* __restrict__ h32,
                                                       const WT* __restrict__ wr,
                                                       const WT* __restrict__ wseg, int T,
                                                       int H, int E, int E1, int kslice,
                                                       float* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e0 = blockIdx.x * RT_EPB + wave * 4;
  const int t0 = blockIdx.y * RT_TT;
  const int s = blockIdx.z;
  if (e0 >= E1) return;
  const int kb = s * kslice;
  const int ke = min(H, kb + kslice);
  const WT* wrow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int e = e0 + j;
    wrow[j] = (e < E) ? wr + (size_t)e * H : ((e == E && wseg) ? wseg : wr);
  }
  const int nt = min(RT_TT, T - t0);
  float acc[RT_TT][4];
#pragma unroll
  for (int t = 0; t < RT_TT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[t][j] = 0.f;

  for (int k = kb + lane * 4; k < ke; k += RT_KCH) {
    float4 wv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wv[j] = rt_load4<WT>(wrow[j] + k);
#pragma unroll
    for (int t = 0; t < RT_TT; ++t) {
      if (t < nt) {
        float4 hv = *(const float4*)(h32 + (size_t)(t0 + t) * H + k);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float a = acc[t][j];
          a = fmaf(hv.x, wv[j].x, a);
          a = fmaf(hv.y, wv[j].y, a);
          a = fmaf(hv.z, wv[j].z, a);
          a = fmaf(hv.w, wv[j].w, a);
          acc[t][j] = a;
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < RT_TT; ++t) {
    if (t < nt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = mx_wave_sum(acc[t][j]);
        if (lane == 0 && e0 + j < E1) out[((size_t)s * T + t0 + t) * E1 + e0 + j] = v;
      }
    }
  }
}

// Number of H-slices the router uses for T tokens (a pure function of the shape).
int mx_router_splits_for(int tokens, int hidden, int e1) {
  int eblocks = mx_ceil_div(e1, RT_EPB);
  int tblocks = mx_ceil_div(tokens > 0 ? tokens : 1, RT_TT);
  int kch = mx_ceil_div(hidden, RT_KCH);
  int s = 1;
  while (eblocks * tblocks * s < 256 && s * 2 <= kch) s *= 2;
  int per = mx_ceil_div(kch, s);
  return mx_ceil_div(kch, per);
}

static int router_kslice(int hidden, int splits) {
  int kch = mx_ceil_div(hidden, RT_KCH);
  return mx_ceil_div(kch, splits) * RT_KCH;
}

extern "C" int mx_router_logits(const float* h32, const void* router_w, const void* shared_gate_w,
                                int32_t param_dtype, int32_t tokens, int32_t hidden,
                                int32_t n_experts, int32_t splits, float* logits, void* stream) {
  if (!h32 || !router_w || !logits || tokens < 0 || hidden <= 0 || n_experts <= 0)
    return MX_ERR_INVALID;
  if (hidden % 4 != 0) return MX_ERR_UNSUPPORTED;
  if (param_dtype != MX_DT_F32 && param_dtype != MX_DT_F16) return MX_ERR_INVALID;
  if (splits < 1) return MX_ERR_INVALID;
  // float4 / 4 x fp16 vector loads of the router rows and of h32.
  const uintptr_t walign = param_dtype == MX_DT_F16 ? 7u : 15u;
  if (((uintptr_t)router_w & walign) || ((uintptr_t)shared_gate_w & walign) ||
      ((uintptr_t)h32 & 15u))
    return MX_ERR_ALIGNMENT;
  if (tokens == 0) return MX_OK;
  const int kslice = router_kslice(hidden, splits);
  if (mx_ceil_div(hidden, kslice) != splits) return MX_ERR_INVALID;
  const int e1 = n_experts + (shared_gate_w ? 1 : 0);
  dim3 grid(mx_ceil_div(e1, RT_EPB), mx_ceil_div(tokens, RT_TT), splits);
  mx_clear_error();
  hipStream_t s = (hipStream_t)stream;
  if (param_dtype == MX_DT_F16)
    hipLaunchKernelGGL(k_router_logits<half_t>, grid, dim3(256), 0, s, h32,
                       (const half_t*)router_w, (const half_t*)shared_gate_w, (int)tokens,
                       (int)hidden, (int)n_experts, e1, kslice, logits);
  else
    hipLaunchKernelGGL(k_router_logits<float>, grid, dim3(256), 0, s, h32,
                       (const float*)router_w, (const float*)shared_gate_w, (int)tokens,
                       (int)hidden, (int)n_experts, e1, kslice, logits);
  return mx_launch_status();
}

// ------------------------------------------------------------------------------------
// Top-k: one wave per token; lane l holds experts l, l+64, ...
//   REF_SOFTMAX_BIAS: z = l + b, p = softmax(z), select on z (= order of p), weight p.
//   SIGMOID_SELECT_BIAS: s = sigmoid(l), select on s + b, weight s.
//   SOFTMAX: z = l, p = softmax(z), select on z, weight p.
// k rounds of a wave-wide arg-max (ties -> lower expert id) give the ids already sorted
// by descending key, as argpartition + argsort(-w) leave them (glm4_moe.py:189-195).
// Then w /= (sum(w) + 1e-20) when norm_topk_prob and w *= routed_scaling.
// ------------------------------------------------------------------------------------
#define TK_MAXK 32

template <int VPT>
__global__ __launch_bounds__(256) void k_router_topk(
    const float* __restrict__ logits, int S, const void* __restrict__ bias, int pdt, int T,
    int E, int E1, int k, int mode, int norm, float scaling, int has_seg,
    int* __restrict__ ids, float* __restrict__ tw, float* __restrict__ shared_w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
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
    const float w = norm ? my_w / (sum + 1e-20f) : my_w;
    ids[(size_t)t * k + lane] = my_id;
    tw[(size_t)t * k + lane] = w * scaling;
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
    }
  }
}

extern "C" int mx_router_topk(const float* logits, int32_t splits, const void* bias,
                              int32_t param_dtype, int32_t tokens, int32_t n_experts,
                              int32_t top_k, int32_t router_mode, int32_t norm_topk_prob,
                              float routed_scaling, int32_t has_shared_gate, int32_t* topk_ids,
                              float* topk_w, float* shared_w, void* stream) {
  if (!logits || !topk_ids || !topk_w || tokens < 0 || n_experts <= 0 || splits < 1)
    return MX_ERR_INVALID;
  if (top_k < 1 || top_k > TK_MAXK || top_k > n_experts) return MX_ERR_INVALID;
  if (router_mode < 0 || router_mode > 2) return MX_ERR_INVALID;
  if (param_dtype != MX_DT_F32 && param_dtype != MX_DT_F16) return MX_ERR_INVALID;
  if (n_experts > 64 * 16) return MX_ERR_UNSUPPORTED;
  if (tokens == 0) return MX_OK;
  const int e1 = n_experts + (has_shared_gate ? 1 : 0);
  const void* b = (router_mode == MX_ROUTER_SOFTMAX) ? nullptr : bias;
  dim3 grid(mx_ceil_div(tokens, 4));
  mx_clear_error();
  hipStream_t s = (hipStream_t)stream;
  const int vpt = mx_ceil_div(n_experts, 64);
#define TK_LAUNCH(V)                                                                       \
  hipLaunchKernelGGL(k_router_topk<V>, grid, dim3(256), 0, s, logits, (int)splits, b,      \
                     (int)param_dtype, (int)tokens, (int)n_experts, e1, (int)top_k,        \
                     (int)router_mode, (int)norm_topk_prob, routed_scaling,                \
                     (int)has_shared_gate, topk_ids, topk_w, shared_w)
  if (vpt <= 1) TK_LAUNCH(1);
  else if (vpt <= 2) TK_LAUNCH(2);
  else if (vpt <= 4) TK_LAUNCH(4);
  else if (vpt <= 8) TK_LAUNCH(8);
  else TK_LAUNCH(16);
#undef TK_LAUNCH
  return mx_launch_status();
}
