// RMSNorm, router logits and router top-k for the MoE block.
//
// Reference: offload_runtime/executors/glm4_moe.py:177-200 (GLM4-MoE) and
// offload_runtime/executors/qwen3_next.py:274-293, :327-329 (Qwen3-Next), with the
// primitives rms_norm / softmax of offload_runtime/executors/_common.py:73-75, :87-90.
// All arithmetic is fp32, as in the NumPy reference (fp16 parameters are widened first).
#include <math.h>

#include "mx_common.h"
#include "mx_internal.h"
#include "mx_route_dev.h"

// ------------------------------------------------------------------------------------
// RMSNorm: one 256-thread block per token.  h = w * (x / sqrt(mean(x^2) + eps)).
// VEC: each thread keeps its float4 slices of the row in registers (H <= 256 * 4 * RN_V),
// so all loads of a row are in flight together.  (One wave per token, four tokens per
// block, measured slower for Qwen3-Next's H = 2048: 28 -> 32 us at 4096 tokens.)  Outputs:
// h32 (fp32; left out when null), h16 = fp16(h) and,
// for the split-plane router GEMM, h16lo = fp16((h - h16) * 2^11) (h - h16 is exact in
// fp32, and so is the power-of-two scaling).  With the split-plane router the launch has
// E x ceil(H / 1024) more blocks, dispatched first, each writing the planes hi = fp16(w),
// lo = fp16((w - hi) * 2^11) of 1024 elements of one router row for the router GEMM, and
// with a shared-expert gate row (qwen3_next.py:328) each token's block also writes the
// gate logit h . w_sg (fp32 products and sums) into column E of the logit slices, so the
// GEMM does not spend a 128-column tile on that one row.
// ------------------------------------------------------------------------------------
#define RN_V 8

// Block sum of the per-thread gate partials (after the block's use of red for the sum of
// squares), then token t's gate logit into slice 0 and zeros into the other slices.
__device__ __forceinline__ void gate_logit_store(const MxRouterSplitW& rs, int t, float gdot,
                                                 float* red) {
  gdot = mx_wave_sum(gdot);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = gdot;
  __syncthreads();
  if (threadIdx.x < rs.S) {
    const float g = threadIdx.x == 0 ? (red[0] + red[1]) + (red[2] + red[3]) : 0.f;
    rs.gate_out[threadIdx.x * rs.gate_slice + (long)t * rs.gate_ld] = g;
  }
}

template <bool VEC>
__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x,
                                                 const void* __restrict__ w, int wdt,
                                                 float eps, int H, float* __restrict__ h32,
                                                 half_t* __restrict__ h16,
                                                 half_t* __restrict__ h16lo, int nsplit,
                                                 MxRouterSplitW rs) {
  if ((int)blockIdx.x < nsplit) {  // 1024 elements of one router row's planes
    const int pieces = (H + 1023) >> 10;
    const int e = blockIdx.x / pieces;
    const int c0 = (blockIdx.x - e * pieces) * 1024;
    const void* src = rs.wr;
    const int base = e * H;
    half_t* hi = rs.whi + (size_t)e * H;
    half_t* lo = rs.wlo + (size_t)e * H;
    if constexpr (VEC) {  // 4 consecutive elements per thread (H % 4 == 0, aligned rows)
      const int i = c0 + 4 * threadIdx.x;
      if (i < H) {
        const float4 v = mx_load_param4(src, rs.pdt, base + i);
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 vh = (h4){(half_t)v.x, (half_t)v.y, (half_t)v.z, (half_t)v.w};
        *(h4*)(hi + i) = vh;
        *(h4*)(lo + i) = (h4){(half_t)((v.x - (float)vh[0]) * 2048.f),
                              (half_t)((v.y - (float)vh[1]) * 2048.f),
                              (half_t)((v.z - (float)vh[2]) * 2048.f),
                              (half_t)((v.w - (float)vh[3]) * 2048.f)};
      }
      return;
    }
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = c0 + threadIdx.x + 256 * u;
      v[u] = i < H ? mx_load_param(src, rs.pdt, base + i) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = c0 + threadIdx.x + 256 * u;
      if (i < H) {
        const half_t vh = (half_t)v[u];
        hi[i] = vh;
        lo[i] = (half_t)((v[u] - (float)vh) * 2048.f);
      }
    }
    return;
  }
  const int t = blockIdx.x - nsplit;
  const float* xr = x + (size_t)t * H;
  float* hr = h32 ? h32 + (size_t)t * H : nullptr;
  half_t* hr16 = h16 ? h16 + (size_t)t * H : nullptr;
  half_t* hrlo = h16lo ? h16lo + (size_t)t * H : nullptr;
  __shared__ float red[4];
  if constexpr (VEC) {
    float4 v[RN_V];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < RN_V; ++i) {
      const int c = (threadIdx.x + 256 * i) * 4;
      v[i] = c < H ? *(const float4*)(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < RN_V; ++i) {
      ss = fmaf(v[i].x, v[i].x, ss);
      ss = fmaf(v[i].y, v[i].y, ss);
      ss = fmaf(v[i].z, v[i].z, ss);
      ss = fmaf(v[i].w, v[i].w, ss);
    }
    ss = mx_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(ss / (float)H + eps);
    float gdot = 0.f;
#pragma unroll
    for (int i = 0; i < RN_V; ++i) {
      const int c = (threadIdx.x + 256 * i) * 4;
      if (c < H) {
        const float4 nw = mx_load_param4(w, wdt, c);
        float4 o;
        o.x = nw.x * (v[i].x / rms);
        o.y = nw.y * (v[i].y / rms);
        o.z = nw.z * (v[i].z / rms);
        o.w = nw.w * (v[i].w / rms);
        if (hr) *(float4*)(hr + c) = o;
        if (rs.gate_out) {
          const float4 g = mx_load_param4(rs.wsg, rs.pdt, c);
          gdot = fmaf(o.x, g.x, gdot);
          gdot = fmaf(o.y, g.y, gdot);
          gdot = fmaf(o.z, g.z, gdot);
          gdot = fmaf(o.w, g.w, gdot);
        }
        if (hr16) {
          typedef _Float16 h4 __attribute__((ext_vector_type(4)));
          const h4 hi = (h4){(half_t)o.x, (half_t)o.y, (half_t)o.z, (half_t)o.w};
          *(h4*)(hr16 + c) = hi;
          if (hrlo)
            *(h4*)(hrlo + c) = (h4){(half_t)((o.x - (float)hi[0]) * 2048.f),
                                    (half_t)((o.y - (float)hi[1]) * 2048.f),
                                    (half_t)((o.z - (float)hi[2]) * 2048.f),
                                    (half_t)((o.w - (float)hi[3]) * 2048.f)};
        }
      }
    }
    if (rs.gate_out) gate_logit_store(rs, t, gdot, red);
  } else {
    float ss = 0.f;
    for (int i = threadIdx.x; i < H; i += 256) {
      float v = xr[i];
      ss = fmaf(v, v, ss);
    }
    ss = mx_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(ss / (float)H + eps);
    float gdot = 0.f;
    for (int i = threadIdx.x; i < H; i += 256) {
      float v = mx_load_param(w, wdt, i) * (xr[i] / rms);
      if (hr) hr[i] = v;
      if (rs.gate_out) gdot = fmaf(v, mx_load_param(rs.wsg, rs.pdt, i), gdot);
      if (hr16) {
        const half_t hi = (half_t)v;
        hr16[i] = hi;
        if (hrlo) hrlo[i] = (half_t)((v - (float)hi) * 2048.f);
      }
    }
    if (rs.gate_out) gate_logit_store(rs, t, gdot, red);
  }
}

int mx_rmsnorm_launch(const float* x, const void* norm_w, int param_dtype, float eps, int tokens,
                      int hidden, float* h32, void* h16, hipStream_t s, void* h16lo,
                      const MxRouterSplitW* rsw) {
  if (h16lo && !h16) return MX_ERR_INVALID;
  MxRouterSplitW rs{};
  if (rsw) {
    rs = *rsw;
    if (!rs.wr || !rs.whi || !rs.wlo || rs.E < 1 || (rs.gate_out && (!rs.wsg || rs.S < 1)))
      return MX_ERR_INVALID;
  }
  if (!h32 && !h16) return MX_ERR_INVALID;
  const int nsplit = rsw ? rs.E * ((hidden + 1023) >> 10) : 0;
  const unsigned grid = (unsigned)tokens + (unsigned)nsplit;
  // Vector path: 4 consecutive elements per load, for x, h and the parameters alike.
  const uintptr_t pal = param_dtype == MX_DT_F16 ? 7u : 15u;
  const uintptr_t sal = rsw && rs.pdt == MX_DT_F16 ? 7u : 15u;
  const bool vec = hidden % 4 == 0 && hidden <= 256 * 4 * RN_V && mx_aligned16(x) &&
                   (!h32 || mx_aligned16(h32)) && (!h16 || ((uintptr_t)h16 & 7u) == 0) &&
                   (!h16lo || ((uintptr_t)h16lo & 7u) == 0) && !((uintptr_t)norm_w & pal) &&
                   (!rsw || (!((uintptr_t)rs.wr & sal) && !((uintptr_t)rs.wsg & sal) &&
                             !((uintptr_t)rs.whi & 7u) && !((uintptr_t)rs.wlo & 7u)));
  mx_clear_error();
  if (vec)
    hipLaunchKernelGGL(k_rmsnorm<true>, dim3(grid), dim3(256), 0, s, x, norm_w, param_dtype, eps,
                       hidden, h32, (half_t*)h16, (half_t*)h16lo, nsplit, rs);
  else
    hipLaunchKernelGGL(k_rmsnorm<false>, dim3(grid), dim3(256), 0, s, x, norm_w, param_dtype,
                       eps, hidden, h32, (half_t*)h16, (half_t*)h16lo, nsplit, rs);
  return mx_launch_status();
}

extern "C" int mx_rmsnorm(const float* x, const void* norm_w, int32_t param_dtype, float eps,
                          int32_t tokens, int32_t hidden, float* h32, void* h16, void* stream) {
  if (!x || !norm_w || !h32 || tokens < 0 || hidden <= 0) return MX_ERR_INVALID;
  if (param_dtype != MX_DT_F32 && param_dtype != MX_DT_F16) return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  return mx_rmsnorm_launch(x, norm_w, param_dtype, eps, tokens, hidden, h32, h16,
                           (hipStream_t)stream);
}

// ------------------------------------------------------------------------------------
// Router logits on fp32 MFMA (v_mfma_f32_16x16x4_f32: full fp32 products and sums).
// Block = 4 waves over a 256-token x 32-expert tile; wave w takes tokens w * 64.. and
// the block's 32 experts, i.e. 4 x 2 fragments of 16 x 16.  (Measured on MI355X against
// 2 x 2 fragments per wave over 64 x 64 tiles: Qwen3-Next 4096 tokens 154 -> 133 us,
// GLM-4.7 2048 tokens 76 -> 63 us; wider expert tiles or deeper load batches were slower.)
// Row e == E is the Qwen3-Next shared-expert gate (qwen3_next.py:328), which rides along
// as an extra "expert".  Grid z splits H into slices; out[s][t][e] holds the partial sum
// of slice s and the top-k kernel adds the slices in ascending order, so the result does
// not depend on scheduling.
//
// Per 16-column chunk lane (i, q) loads 4 consecutive columns 4q .. 4q+3 of its token
// row and of its expert row (float4); MFMA e (0..3) takes element e of both, so the
// four MFMAs cover the chunk's 16 columns once each.  Loads are clamped in bounds and
// masked (branch-free), and a chunk batch is in flight while the previous one runs.
// ------------------------------------------------------------------------------------
#ifndef RT_KCH
#define RT_KCH 256  // H-slice granularity of the prefill router (elements)
#endif

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

#ifndef RM_UK
#define RM_UK 1  // chunks per load batch (two batches in flight)
#endif
// Block shape: each wave computes RT_FA x RT_FB fragments of 16 x 16 (tokens x experts);
// the 4 waves of a block are RT_WA along tokens by 4 / RT_WA along experts.
#ifndef RT_FA
#define RT_FA 4
#endif
#ifndef RT_FB
#define RT_FB 2
#endif
#ifndef RT_WA
#define RT_WA 4
#endif
constexpr int RT_BT = 16 * RT_FA * RT_WA;        // tokens per block
constexpr int RT_BE = 16 * RT_FB * (4 / RT_WA);  // experts per block

#ifndef RT_WPE
#define RT_WPE 4  // waves per SIMD the prefill router is compiled for
#endif

template <typename WT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, RT_WPE))) void
k_router_logits(const float* __restrict__ h32, const WT* __restrict__ wr,
                const WT* __restrict__ wseg, int T, int H, int E, int E1, int kslice,
                float* __restrict__ out) {
  constexpr int FA = RT_FA, FB = RT_FB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  const int t0 = blockIdx.x * RT_BT + (wave % RT_WA) * 16 * FA;
  const int e0 = blockIdx.y * RT_BE + (wave / RT_WA) * 16 * FB;
  const int s = blockIdx.z;
  const int kb = s * kslice, ke = min(H, kb + kslice);
  if (kb >= ke) return;
  const float* arow[FA];
  const WT* brow[FB];
#pragma unroll
  for (int a = 0; a < FA; ++a) arow[a] = h32 + (size_t)min(t0 + 16 * a + j, T - 1) * H;
#pragma unroll
  for (int b = 0; b < FB; ++b) {
    const int e = e0 + 16 * b + j;
    brow[b] = e < E ? wr + (size_t)e * H : ((e == E && wseg) ? wseg : wr + (size_t)(E - 1) * H);
  }
  float4_t acc[FA][FB];
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b) acc[a][b] = (float4_t){0.f, 0.f, 0.f, 0.f};

  const int nch = (ke - kb + 15) / 16;
  auto load = [&](int c, float4 (&av)[FA], float4 (&bv)[FB]) {
    const int k = kb + 16 * c + 4 * q;
    const bool in = k < ke;
    const int kk = in ? k : ke - 4;  // clamped in bounds, masked below
#pragma unroll
    for (int a = 0; a < FA; ++a) {
      const float4 v = *(const float4*)(arow[a] + kk);
      av[a] = in ? v : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const float4 v = rt_load4<WT>(brow[b] + kk);
      bv[b] = in ? v : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto mma = [&](const float4 (&av)[FA], const float4 (&bv)[FB]) {
#pragma unroll
    for (int a = 0; a < FA; ++a)
#pragma unroll
      for (int b = 0; b < FB; ++b) {
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].x, bv[b].x, acc[a][b], 0, 0, 0);
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].y, bv[b].y, acc[a][b], 0, 0, 0);
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].z, bv[b].z, acc[a][b], 0, 0, 0);
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].w, bv[b].w, acc[a][b], 0, 0, 0);
      }
  };
  // Batches of RM_UK chunks, two register sets; the batch count is padded to even and
  // padding chunks read (masked) zeros.
  const int nb = (nch + RM_UK - 1) / RM_UK;
  float4 ax[RM_UK][FA], bx[RM_UK][FB], ay[RM_UK][FA], by[RM_UK][FB];
#pragma unroll
  for (int u = 0; u < RM_UK; ++u) load(u, ax[u], bx[u]);
  for (int bt = 0; bt < nb; bt += 2) {
#pragma unroll
    for (int u = 0; u < RM_UK; ++u) load((bt + 1) * RM_UK + u, ay[u], by[u]);
#pragma unroll
    for (int u = 0; u < RM_UK; ++u) mma(ax[u], bx[u]);
#pragma unroll
    for (int u = 0; u < RM_UK; ++u) load((bt + 2) * RM_UK + u, ax[u], bx[u]);
#pragma unroll
    for (int u = 0; u < RM_UK; ++u) mma(ay[u], by[u]);
  }
#pragma unroll
  for (int a = 0; a < FA; ++a)
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const int e = e0 + 16 * b + j;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + 16 * a + 4 * q + r;
        if (t < T && e < E1) out[((size_t)s * T + t) * E1 + e] = acc[a][b][r];
      }
    }
}

// Router logits of long inputs run on the LDS-staged GEMM (mx_dense_gemm.hip), the
// reduction cut into slices over gridDim.y:
//  * RT_SPLIT: inside the MoE block, where h16 = fp16(h) exists: h and the router rows as
//    two fp16 planes each (mx_gemm_f16x2_slices; the block's RMSNorm writes the low plane of
//    h, mx_router_split_weights the planes of the router rows and the shared-expert gate
//    row, one [E1, H] matrix); 256 x 128 tiles, one block per CU, slices of a multiple of
//    32 columns.
//  * RT_GEMM32: fp32 router rows otherwise (mx_gemm_f32_slices; the routed rows and the
//    gate row as two weight segments); 128 x 128 tiles, two blocks per CU, slices of a
//    multiple of 16 columns.
// Other inputs run k_router_logits above (slices of RT_KCH columns).
#ifndef RT_GEMM_MIN_TOKENS
#define RT_GEMM_MIN_TOKENS 65
#endif
#ifndef RT_USE_SPLIT
#define RT_USE_SPLIT 1
#endif
#ifndef RT_SPLIT_FILL
#define RT_SPLIT_FILL 256  // blocks of one round of the split-plane GEMM (one per CU)
#endif
#ifndef RT_SPLIT_ROUTED
#define RT_SPLIT_ROUTED 1  // split-plane slice count from the routed rows' tiles
#endif
static bool router_on_gemm(int tokens, int hidden, int e1, int param_dtype) {
  return param_dtype == MX_DT_F32 && tokens >= RT_GEMM_MIN_TOKENS && hidden % MX_GEMM_KMULT_F32 == 0 &&
         (long)tokens * hidden * 4 < (1l << 31) && (long)e1 * hidden * 4 < (1l << 31);
}
bool mx_router_on_split(int tokens, int hidden, int e1, int weight_dtype) {
  return RT_USE_SPLIT && weight_dtype != MX_DT_F32 && tokens >= RT_GEMM_MIN_TOKENS &&
         hidden % MX_GEMM_KMULT_F16 == 0 && (long)tokens * hidden * 2 < (1l << 31) &&
         (long)e1 * hidden * 2 < (1l << 31);
}

// Number of H-slices the router uses for T tokens (a pure function of the shape), at most
// 16 and at most one per RT_KCH columns (k_router_logits) or per GEMM stage width
// (MX_GEMM_KMULT_F32 columns on the fp32 GEMM, MX_GEMM_KMULT_F16 on the split-plane GEMM;
// weight_dtype < 0: outside the MoE block, no split planes).
int mx_router_splits_for(int tokens, int hidden, int n_experts, int has_shared_gate,
                         int param_dtype, int weight_dtype) {
  const int t = tokens > 0 ? tokens : 1;
  const int e1 = n_experts + (has_shared_gate ? 1 : 0);
  long tiles, fill;
  int kch;
  if (weight_dtype >= 0 && mx_router_on_split(t, hidden, e1, weight_dtype)) {
    // Largest slice count whose blocks fit one round at one block per CU.  The GEMM covers
    // the routed rows only (the RMSNorm launch computes the shared-expert gate logit).
    // Qwen3-Next, 4096 tokens: 32 x 4 tiles x 2 slices; GLM-4.7, 2048 tokens: 16 x 2 x 8.
    const int cols = RT_SPLIT_ROUTED ? n_experts : e1;
    tiles = (long)mx_ceil_div(t, MX_GEMM_SPLIT_BM) * mx_ceil_div(cols, MX_GEMM_SPLIT_BN);
    fill = RT_SPLIT_FILL;
    kch = hidden / MX_GEMM_KMULT_F16;
  } else if (router_on_gemm(t, hidden, e1, param_dtype)) {
    // Largest slice count whose blocks fit one round at two blocks per CU.  Qwen3-Next,
    // 4096 tokens: 32 x (4 + 1) tiles x 3 slices; GLM-4.7, 2048 tokens: 16 x 2 x 16.
    tiles = (long)mx_ceil_div(t, 128) *
            (mx_ceil_div(n_experts, 128) + (has_shared_gate ? 1 : 0));
    fill = 512;
    kch = hidden / MX_GEMM_KMULT_F32;
  } else {
    // Largest slice count whose blocks fit one round at 4 waves per SIMD (1024 blocks of 4
    // waves on 256 CUs).
    tiles = (long)mx_ceil_div(t, RT_BT) * mx_ceil_div(e1, RT_BE);
    fill = 1024;
    kch = mx_ceil_div(hidden, RT_KCH);
  }
  int s = 1;
  while (tiles * (s + 1) <= fill && s + 1 <= kch && s < 16) ++s;
  const int per = mx_ceil_div(kch, s);
  return mx_ceil_div(kch, per);
}

static int router_kslice(int hidden, int splits) {
  int kch = mx_ceil_div(hidden, RT_KCH);
  return mx_ceil_div(kch, splits) * RT_KCH;
}

size_t mx_router_split_bytes(int hidden, int e1) { return mx_align_up((size_t)e1 * hidden * 2, 256) * 2; }

MxRouterSplitW mx_router_split_planes(const void* router_w, const void* shared_gate_w,
                                      int param_dtype, int n_experts, int hidden, int tokens,
                                      int splits, void* wsplit, float* logits) {
  const int e1 = n_experts + (shared_gate_w ? 1 : 0);
  MxRouterSplitW r{};
  r.wr = router_w;
  r.pdt = param_dtype;
  r.E = n_experts;
  r.whi = (half_t*)wsplit;
  r.wlo = (half_t*)((char*)wsplit + mx_align_up((size_t)e1 * hidden * 2, 256));
  if (shared_gate_w) {
    r.wsg = shared_gate_w;
    r.gate_out = logits + n_experts;
    r.gate_ld = e1;
    r.gate_slice = (long)tokens * e1;
    r.S = splits;
  }
  return r;
}

int mx_router_logits_split(const void* h16, const void* h16lo, const void* router_w,
                           const void* shared_gate_w, int param_dtype, int tokens, int hidden,
                           int n_experts, int splits, void* wsplit, float* logits, hipStream_t s) {
  if (!h16 || !h16lo || !router_w || !wsplit || !logits || tokens <= 0 || hidden <= 0 ||
      n_experts <= 0 || splits < 1)
    return MX_ERR_INVALID;
  const int e1 = n_experts + (shared_gate_w ? 1 : 0);
  if (!mx_router_on_split(tokens, hidden, e1, MX_DT_F16)) return MX_ERR_UNSUPPORTED;
  const int kslice = mx_ceil_div(hidden / MX_GEMM_KMULT_F16, splits) * MX_GEMM_KMULT_F16;
  if (mx_ceil_div(hidden, kslice) != splits) return MX_ERR_INVALID;
  const MxRouterSplitW r = mx_router_split_planes(router_w, shared_gate_w, param_dtype,
                                                  n_experts, hidden, tokens, splits, wsplit,
                                                  logits);
  // Routed rows only: the shared-expert gate logit (column E) comes from the RMSNorm launch.
  MxGemmSeg g{r.whi, logits, n_experts, e1};
  g.w_lo = r.wlo;
  return mx_gemm_f16x2_slices(h16, h16lo, tokens, hidden, &g, 1, kslice, (long)tokens * e1, s);
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
  const int e1 = n_experts + (shared_gate_w ? 1 : 0);
  hipStream_t s = (hipStream_t)stream;
  if (router_on_gemm(tokens, hidden, e1, param_dtype)) {
    const int kslice = mx_ceil_div(hidden / MX_GEMM_KMULT_F32, splits) * MX_GEMM_KMULT_F32;
    if (mx_ceil_div(hidden, kslice) != splits) return MX_ERR_INVALID;
    const MxGemmSeg g[2] = {{router_w, logits, n_experts, e1},
                            {shared_gate_w, logits + n_experts, 1, e1}};
    return mx_gemm_f32_slices(h32, tokens, hidden, g, shared_gate_w ? 2 : 1, kslice,
                              (long)tokens * e1, s);
  }
  const int kslice = router_kslice(hidden, splits);
  if (mx_ceil_div(hidden, kslice) != splits) return MX_ERR_INVALID;
  dim3 grid(mx_ceil_div(tokens, RT_BT), mx_ceil_div(e1, RT_BE), splits);
  mx_clear_error();
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
template <int VPT>
__global__ __launch_bounds__(256) void k_router_topk(
    const float* __restrict__ logits, int S, const void* __restrict__ bias, int pdt, int T,
    int E, int E1, int k, int mode, int norm, float scaling, int has_seg,
    int* __restrict__ ids, float* __restrict__ tw, float* __restrict__ shared_w) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  mx_topk_token<VPT>(logits, S, T, t, bias, pdt, E, E1, k, mode, norm, scaling, has_seg, ids,
                     tw, shared_w);
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
  else if (vpt <= 3) TK_LAUNCH(3);
  else if (vpt <= 4) TK_LAUNCH(4);
  else if (vpt <= 6) TK_LAUNCH(6);
  else if (vpt <= 8) TK_LAUNCH(8);
  else if (vpt <= 12) TK_LAUNCH(12);
  else TK_LAUNCH(16);
#undef TK_LAUNCH
  return mx_launch_status();
}

// ------------------------------------------------------------------------------------
// Decode router (T <= 64): two launches, the RMSNorm folded into the first.
//   k_router_logits_decode: one block per (expert row, group of up to 8 tokens) over the
//     full H (no H split); also writes the normalised activations.
//   k_topk_dispatch: one workgroup of up to 16 waves; per-token top-k (one wave per
//     token), then the dispatch.  A kernel boundary separates the two: the blocks of the
//     logits kernel run on every XCD, and publishing their results inside one launch
//     would need an L2 write-back per block.
// ------------------------------------------------------------------------------------
// Block (e, g): expert row e (row E = Qwen3-Next shared gate) against tokens g*TT ..
// g*TT+TT-1, with the RMSNorm folded in: each lane accumulates x . (norm_w * w_e) and
// x . x over its H columns, the 4 waves (H quarters) are added in LDS in a fixed order,
// and logit = dot / rms with rms = sqrt(mean(x^2) + eps) (_common.py:73-75).  The blocks
// also write the normalised rows h = norm_w * (x / rms) (fp32, and fp16 when h16 is
// given) for the expert kernels.  Rows past the last token re-read the last token
// (results discarded), so the loop body is branch-free and its loads issue together.
// At most 2 waves per SIMD: the register budget lets every load of a loop step be
// issued before the first FMA waits (at the default occupancy target the compiler
// serialises load -> wait -> FMA per token row).
template <typename WT, int TT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void
k_router_logits_decode(
    const float* __restrict__ x, const WT* __restrict__ norm_w, float eps,
    const WT* __restrict__ wr, const WT* __restrict__ wseg, int T, int H, int E, int E1,
    float* __restrict__ logits, float* __restrict__ h32, half_t* __restrict__ h16) {
  __shared__ float part[4][TT], sq[4][TT];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x;
  const int t0 = blockIdx.y * TT;
  const WT* row = (e < E) ? wr + (size_t)e * H : wseg;
  // One sweep of the wave covers 64 lanes x 4 columns; the loop stride is that sweep and
  // does not follow the prefill router's slice width.
  constexpr int SWEEP = 64 * 4;
  const int hq = (H / 4 + SWEEP - 1) / SWEEP * SWEEP;  // H quarter per wave, whole sweeps
  const int kb = wave * hq, ke = min(H, kb + hq);
  float acc[TT], ss[TT];
  const float* xrow[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    acc[t] = 0.f;
    ss[t] = 0.f;
    xrow[t] = x + (size_t)min(t0 + t, T - 1) * H;
  }
#pragma unroll 4
  for (int c = kb + lane * 4; c < ke; c += SWEEP) {
    const float4 wv = rt_load4<WT>(row + c);
    const float4 nv = rt_load4<WT>(norm_w + c);
    const float4 g = make_float4(nv.x * wv.x, nv.y * wv.y, nv.z * wv.z, nv.w * wv.w);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const float4 xv = *(const float4*)(xrow[t] + c);
      float a = acc[t], q = ss[t];
      a = fmaf(xv.x, g.x, a);
      q = fmaf(xv.x, xv.x, q);
      a = fmaf(xv.y, g.y, a);
      q = fmaf(xv.y, xv.y, q);
      a = fmaf(xv.z, g.z, a);
      q = fmaf(xv.z, xv.z, q);
      a = fmaf(xv.w, g.w, a);
      q = fmaf(xv.w, xv.w, q);
      acc[t] = a;
      ss[t] = q;
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const float v = mx_wave_sum(acc[t]);
    const float q = mx_wave_sum(ss[t]);
    if (lane == 0) {
      part[wave][t] = v;
      sq[wave][t] = q;
    }
  }
  __syncthreads();
  if (threadIdx.x < TT && t0 + (int)threadIdx.x < T) {
    const int t = threadIdx.x;
    const float rms = sqrtf(((sq[0][t] + sq[1][t]) + (sq[2][t] + sq[3][t])) / (float)H + eps);
    logits[(size_t)(t0 + t) * E1 + e] = ((part[0][t] + part[1][t]) + (part[2][t] + part[3][t])) / rms;
  }
  // Normalised rows of this token group, spread over all blocks of the group: one
  // float4 per thread (the x reads hit L2).  Every block reduced the same values in the
  // same order, so all of them hold the same rms.
  const int ng = min(TT, T - t0), h4 = H / 4;
  for (int i = e * 256 + (int)threadIdx.x; i < ng * h4; i += E1 * 256) {
    const int t = i / h4, c = (i - t * h4) * 4;
    const float rms = sqrtf(((sq[0][t] + sq[1][t]) + (sq[2][t] + sq[3][t])) / (float)H + eps);
    const size_t o = (size_t)(t0 + t) * H + c;
    const float4 xv = *(const float4*)(x + o);
    const float4 nv = rt_load4<WT>(norm_w + c);
    const float4 hv = make_float4(nv.x * (xv.x / rms), nv.y * (xv.y / rms), nv.z * (xv.z / rms),
                                  nv.w * (xv.w / rms));
    *(float4*)(h32 + o) = hv;
    if (h16) {
      typedef _Float16 h4v __attribute__((ext_vector_type(4)));
      *(h4v*)(h16 + o) = (h4v){(half_t)hv.x, (half_t)hv.y, (half_t)hv.z, (half_t)hv.w};
    }
  }
}

// 16 waves; 8 for E > 512 (the wider selection state needs the larger register budget).
template <int VPT>
__global__ __launch_bounds__(VPT > 8 ? 512 : 1024) void k_topk_dispatch(
    const float* __restrict__ logits, const void* __restrict__ bias, int pdt, int T, int E,
    int E1, int k, int mode, int norm, float scaling, int has_seg, int has_shared, int m_blk,
    int* __restrict__ ids, float* __restrict__ tw, float* __restrict__ shared_w,
    int* __restrict__ counts, int* __restrict__ offsets, int* __restrict__ sorted_tok,
    float* __restrict__ sorted_w, int* __restrict__ pair_pos, int* __restrict__ g_expert,
    int* __restrict__ g_start, int* __restrict__ g_count, int* __restrict__ n_groups,
    int* __restrict__ mt_group, int* __restrict__ mt_row0, int* __restrict__ n_mtiles) {
  // Dynamic LDS: dispatch tables, then the staged top-k results (ids, weights, shared
  // weights) so the dispatch phases never go back to global memory.
  extern __shared__ __align__(16) unsigned char smem[];
  const int nw = blockDim.x >> 6;
  unsigned char* stage = smem + mx_dispatch_small_lds_bytes(E);
  int* sid = (int*)stage;
  float* sw = (float*)(sid + T * k);
  float* ssw = sw + T * k;
  if (VPT >= 6 && VPT <= 8 && T * VPT <= nw) {
    // Small batch over many experts: VPT = ceil(E / 64) waves per token
    // (mx_topk_par_cand / _final).  Measured on MI355X at 1 token: 512 experts 11.8 ->
    // 10.3 us per launch; with 160 experts the single-wave selection is faster (6.5 vs 7.4).
    __shared__ MxTopkPar par;
    const int wv = threadIdx.x >> 6;
    if (wv < T * VPT) mx_topk_par_cand(par, logits, bias, pdt, E, E1, k, mode, VPT, wv);
    mx_lds_sync();
    if (wv < T)
      mx_topk_par_final<(VPT + 1) / 2>(par, logits, wv, E, E1, k, mode, norm, scaling, VPT,
                                       has_seg, ids, tw, shared_w, sid, sw, ssw);
  } else {
    for (int t = threadIdx.x >> 6; t < T; t += nw)
      mx_topk_token<VPT>(logits, 1, T, t, bias, pdt, E, E1, k, mode, norm, scaling, has_seg,
                         ids, tw, shared_w, sid, sw, ssw);
  }
  if (T == 1) {
    // One token: wave 0 selected it and writes the tables directly.
    if (threadIdx.x >= 64) return;
    mx_lds_fence();
    const int lane = threadIdx.x;
    mx_dispatch_one_token(lane < k ? sid[lane] : 0, lane < k ? sw[lane] : 0.f,
                          shared_w ? ssw[0] : 1.f, k, E, has_shared, counts, offsets, sorted_tok,
                          sorted_w, pair_pos, g_expert, g_start, g_count, n_groups, mt_group,
                          mt_row0, n_mtiles);
    return;
  }
  mx_lds_sync();
  mx_dispatch_block_small(smem, sid, sw, shared_w ? ssw : nullptr, T, k, E, has_shared, m_blk,
                          counts, offsets, sorted_tok, sorted_w, pair_pos, g_expert, g_start,
                          g_count, n_groups, mt_group, mt_row0, n_mtiles);
}

// Dynamic LDS of the top-k/dispatch workgroup: dispatch tables, then the staged top-k
// results (the top-k rows and the small-batch candidates take about 15 KB of static LDS
// besides, so 48 KB of dynamic LDS keeps the workgroup within 64 KB).
static size_t decode_lds_bytes(const MxMoeDesc* d, int T) {
  return mx_dispatch_small_lds_bytes(d->n_experts) + (size_t)T * d->top_k * 8 + (size_t)T * 4;
}

bool mx_one_token_select_ok(const MxMoeDesc* d) {
  return d->n_experts <= MX_SEL_MAX_E && d->n_experts <= 512 && d->top_k <= TK_MAXK;
}

bool mx_router_decode_ok(const MxMoeDesc* d, const MxMoeWeights* w, int T, const float* x) {
  const uintptr_t walign = d->param_dtype == MX_DT_F16 ? 7u : 15u;
  return T >= 1 && T <= 64 && d->n_experts <= 1024 && d->top_k <= MX_DISPATCH_MAXK &&
         d->hidden % 4 == 0 && decode_lds_bytes(d, T) <= 48 * 1024 && mx_aligned16(x) && !((uintptr_t)w->norm_w & walign) &&
         !((uintptr_t)w->router_w & walign) && !((uintptr_t)w->shared_gate_w & walign);
}

int mx_router_decode_launch(const MxMoeDesc* d, const MxMoeWeights* w, int T, const float* x,
                            float* h32, void* h16, float* logits, int* ids, float* tw,
                            float* shared_w, int m_blk, int* counts, int* offsets,
                            int* sorted_tok, float* sorted_w, int* pair_pos, int* g_expert,
                            int* g_start, int* g_count, int* n_groups, int* mt_group,
                            int* mt_row0, int* n_mtiles, hipStream_t s, bool select_later) {
  const int E = d->n_experts, H = d->hidden;
  const int e1 = E + (d->has_shared_gate ? 1 : 0);
  const int has_shared = d->shared_inter > 0;
  if (!mx_router_decode_ok(d, w, T, x)) return MX_ERR_UNSUPPORTED;
  if (select_later && !(T == 1 && mx_one_token_select_ok(d))) return MX_ERR_INVALID;
  const int vpt = mx_ceil_div(E, 64);
  const int nw = vpt > 8 ? 8 : 16;
  const size_t lds = decode_lds_bytes(d, T);
  if (!mx_aligned16(h32) || ((uintptr_t)h16 & 7u)) return MX_ERR_ALIGNMENT;
  const void* b = (d->router_mode == MX_ROUTER_SOFTMAX || !d->has_bias) ? nullptr : w->bias;
  const void* seg = d->has_shared_gate ? w->shared_gate_w : nullptr;
  mx_clear_error();
#define RL_LAUNCH(WT_, TT_)                                                                    \
  hipLaunchKernelGGL((k_router_logits_decode<WT_, TT_>), dim3(e1, mx_ceil_div(T, TT_)),        \
                     dim3(256), 0, s, x, (const WT_*)w->norm_w, d->eps, (const WT_*)w->router_w, \
                     (const WT_*)seg, T, H, E, e1, logits, h32, (half_t*)h16)
#define RL_TT(WT_)                                  \
  if (T <= 1) RL_LAUNCH(WT_, 1);                    \
  else if (T <= 2) RL_LAUNCH(WT_, 2);               \
  else if (T <= 4) RL_LAUNCH(WT_, 4);               \
  else RL_LAUNCH(WT_, 8);
  if (d->param_dtype == MX_DT_F16) {
    RL_TT(half_t)
  } else {
    RL_TT(float)
  }
#undef RL_TT
#undef RL_LAUNCH
  MX_TRY(mx_launch_status());
  if (select_later) return MX_OK;
  // One token with a single-wave selection needs one wave only.
  const int nwl = (T == 1 && vpt < 6) ? 1 : nw;
#define TD_LAUNCH(V)                                                                           \
  hipLaunchKernelGGL((k_topk_dispatch<V>), dim3(1), dim3(64 * nwl), lds, s, logits, b,          \
                     d->param_dtype, T, E, e1, d->top_k, d->router_mode, d->norm_topk_prob,     \
                     d->routed_scaling, d->has_shared_gate, has_shared, m_blk, ids, tw,         \
                     shared_w, counts, offsets, sorted_tok, sorted_w, pair_pos, g_expert,       \
                     g_start, g_count, n_groups, mt_group, mt_row0, n_mtiles)
  if (vpt <= 1) TD_LAUNCH(1);
  else if (vpt <= 2) TD_LAUNCH(2);
  else if (vpt <= 3) TD_LAUNCH(3);
  else if (vpt <= 4) TD_LAUNCH(4);
  else if (vpt <= 6) TD_LAUNCH(6);
  else if (vpt <= 8) TD_LAUNCH(8);
  else if (vpt <= 12) TD_LAUNCH(12);
  else TD_LAUNCH(16);
#undef TD_LAUNCH
  return mx_launch_status();
}
