// Weighted combine + shared expert + residual.
//
// Reference: offload_runtime/executors/glm4_moe.py:203, :227-231, :238, :240 and
// qwen3_next.py:296, :315-318, :331, :333:
//   output = 0; output[tok] += w * expert_out (routed); output = output + shared_out;
//   return x + output.
// The routing weight (and the Qwen3-Next sigmoid gate of the shared expert) is already
// folded into y by the down-projection epilogue, so each token only sums its k routed
// rows (slot order), adds its shared row and the residual.  No atomics: fixed order.
// y rows are fp32, or fp16 after the prefill down launch (k_combine_y16); sums in fp32.
#include "mx_common.h"
#include "mx_internal.h"

typedef float f4v __attribute__((ext_vector_type(4)));

template <bool VEC4>
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ x,
                                                 const float* __restrict__ y,
                                                 const int* __restrict__ pair_pos, int H, int k,
                                                 long shared_row0, float* out) {
  const int t = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * (VEC4 ? 4 : 1);
  if (c >= H) return;
  const int* pp = pair_pos + (size_t)t * k;
  if constexpr (VEC4) {
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    // Slots in groups of 8: all loads of a group are issued before the ordered adds.  Rows
    // of y are read once, with the nontemporal hint (Qwen3-Next 4096 tokens: 89 -> 68 us;
    // GLM-4.7 2048 tokens: 88 -> 74 us).
    for (int j0 = 0; j0 < k; j0 += 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int p = (j0 + u < k) ? pp[j0 + u] : -1;
        const f4v r = p >= 0 ? __builtin_nontemporal_load((const f4v*)(y + (size_t)p * H + c))
                             : (f4v){0.f, 0.f, 0.f, 0.f};
        v[u] = make_float4(r[0], r[1], r[2], r[3]);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        o.x += v[u].x;
        o.y += v[u].y;
        o.z += v[u].z;
        o.w += v[u].w;
      }
    }
    if (shared_row0 >= 0) {
      const float4 v = *(const float4*)(y + (size_t)(shared_row0 + t) * H + c);
      o.x += v.x;
      o.y += v.y;
      o.z += v.z;
      o.w += v.w;
    }
    const float4 xv = *(const float4*)(x + (size_t)t * H + c);
    *(float4*)(out + (size_t)t * H + c) = make_float4(xv.x + o.x, xv.y + o.y, xv.z + o.z, xv.w + o.w);
  } else {
    float o = 0.f;
    for (int j = 0; j < k; ++j) {
      const int p = pp[j];
      if (p >= 0) o += y[(size_t)p * H + c];
    }
    if (shared_row0 >= 0) o += y[(size_t)(shared_row0 + t) * H + c];
    out[(size_t)t * H + c] = x[(size_t)t * H + c] + o;
  }
}

// fp16 y rows (the prefill down launch's output): 8 columns per thread, one 16-byte
// nontemporal load per row and slot; the same fixed order of adds (slots in slot order,
// then the shared row, then the residual), in fp32.
__global__ __launch_bounds__(256) void k_combine_y16(const float* __restrict__ x,
                                                     const half_t* __restrict__ y,
                                                     const int* __restrict__ pair_pos, int H,
                                                     int k, long shared_row0, float* out) {
  typedef _Float16 h8v __attribute__((ext_vector_type(8)));
  const int t = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= H) return;
  const int* pp = pair_pos + (size_t)t * k;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < k; j0 += 8) {
    h8v v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = (j0 + u < k) ? pp[j0 + u] : -1;
      v[u] = p >= 0 ? __builtin_nontemporal_load((const h8v*)(y + (size_t)p * H + c))
                    : (h8v){0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += (float)v[u][e];
  }
  if (shared_row0 >= 0) {
    const h8v v = *(const h8v*)(y + (size_t)(shared_row0 + t) * H + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] += (float)v[e];
  }
  const float4* xr = (const float4*)(x + (size_t)t * H + c);
  float4* orow = (float4*)(out + (size_t)t * H + c);
  const float4 x0 = xr[0], x1 = xr[1];
  orow[0] = make_float4(x0.x + o[0], x0.y + o[1], x0.z + o[2], x0.w + o[3]);
  orow[1] = make_float4(x1.x + o[4], x1.y + o[5], x1.z + o[6], x1.w + o[7]);
}

extern "C" int mx_combine(const float* x, const float* y, const int32_t* pair_pos, int32_t tokens,
                          int32_t hidden, int32_t top_k, int32_t has_shared, float* out,
                          void* stream) {
  return mx_combine_rows(x, y, pair_pos, tokens, hidden, top_k, has_shared, out, false,
                         (hipStream_t)stream);
}

int mx_combine_rows(const float* x, const void* y, const int32_t* pair_pos, int tokens,
                    int hidden, int top_k, int has_shared, float* out, bool y16, hipStream_t s) {
  if (!x || !y || !pair_pos || !out || tokens < 0 || hidden <= 0 || top_k < 1)
    return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  const long shared_row0 = has_shared ? (long)tokens * top_k : -1;
  if (y16) {
    if (hidden % 8) return MX_ERR_UNSUPPORTED;
    if (!mx_aligned16(x) || !mx_aligned16(y) || !mx_aligned16(out)) return MX_ERR_ALIGNMENT;
    mx_clear_error();
    hipLaunchKernelGGL(k_combine_y16, dim3(mx_ceil_div(hidden, 2048), tokens), dim3(256), 0, s,
                       x, (const half_t*)y, pair_pos, (int)hidden, (int)top_k, shared_row0, out);
    return mx_launch_status();
  }
  const bool vec = (hidden % 4 == 0) && mx_aligned16(x) && mx_aligned16(y) && mx_aligned16(out);
  mx_clear_error();
  if (vec)
    hipLaunchKernelGGL(k_combine<true>, dim3(mx_ceil_div(hidden, 1024), tokens), dim3(256), 0, s,
                       x, (const float*)y, pair_pos, (int)hidden, (int)top_k, shared_row0, out);
  else
    hipLaunchKernelGGL(k_combine<false>, dim3(mx_ceil_div(hidden, 256), tokens), dim3(256), 0, s,
                       x, (const float*)y, pair_pos, (int)hidden, (int)top_k, shared_row0, out);
  return mx_launch_status();
}
