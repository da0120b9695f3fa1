// Weighted combine + shared expert + residual.
//
// Reference: offload_runtime/executors/glm4_moe.py:203, :227-231, :238, :240 and
// qwen3_next.py:296, :315-318, :331, :333:
//   output = 0; output[tok] += w * expert_out (routed); output = output + shared_out;
//   return x + output.
// The routing weight (and the Qwen3-Next sigmoid gate of the shared expert) is already
// folded into y by the down-projection epilogue, so each token only sums its k routed
// rows (slot order), adds its shared row and the residual.  No atomics: fixed order.
#include "mx_common.h"

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

extern "C" int mx_combine(const float* x, const float* y, const int32_t* pair_pos, int32_t tokens,
                          int32_t hidden, int32_t top_k, int32_t has_shared, float* out,
                          void* stream) {
  if (!x || !y || !pair_pos || !out || tokens < 0 || hidden <= 0 || top_k < 1)
    return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  const long shared_row0 = has_shared ? (long)tokens * top_k : -1;
  const bool vec = (hidden % 4 == 0) && mx_aligned16(x) && mx_aligned16(y) && mx_aligned16(out);
  mx_clear_error();
  hipStream_t s = (hipStream_t)stream;
  if (vec)
    hipLaunchKernelGGL(k_combine<true>, dim3(mx_ceil_div(hidden, 1024), tokens), dim3(256), 0, s,
                       x, y, pair_pos, (int)hidden, (int)top_k, shared_row0, out);
  else
    hipLaunchKernelGGL(k_combine<false>, dim3(mx_ceil_div(hidden, 256), tokens), dim3(256), 0, s,
                       x, y, pair_pos, (int)hidden, (int)top_k, shared_row0, out);
  return mx_launch_status();
}
