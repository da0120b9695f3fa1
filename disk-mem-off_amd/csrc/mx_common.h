// Shared device helpers for the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_mi355x.h"

typedef _Float16 half_t;
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef int int4_t __attribute__((ext_vector_type(4)));

#define MX_WAVE 64

// Return the status of the last launch (or of a runtime call) as an ABI int.
static inline int mx_status(hipError_t e) { return e == hipSuccess ? MX_OK : (int)e; }
// hipGetLastError() also reports errors left by earlier runtime calls (for example the
// not-ready status of hipEventQuery), so every launch site clears it first.
static inline void mx_clear_error() { (void)hipGetLastError(); }
static inline int mx_launch_status() { return mx_status(hipGetLastError()); }

#define MX_TRY(expr)                      \
  do {                                    \
    int _mx_rc = (expr);                  \
    if (_mx_rc != MX_OK) return _mx_rc;   \
  } while (0)

static inline bool mx_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Load one parameter element (fp32 or fp16 storage) as fp32.
__device__ __forceinline__ float mx_load_param(const void* p, int dtype, int i) {
  return dtype == MX_DT_F16 ? (float)((const half_t*)p)[i] : ((const float*)p)[i];
}
// Elements i .. i + 3 in one load (16-byte aligned fp32 or 8-byte aligned fp16 at i).
__device__ __forceinline__ float4 mx_load_param4(const void* p, int dtype, int i) {
  if (dtype == MX_DT_F16) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 v = *(const h4*)((const half_t*)p + i);
    return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
  }
  return *(const float4*)((const float*)p + i);
}

// Wave reductions: DPP swaps inside each 16-lane row (quad pairs, quads, half-rows), then
// the four row totals are read with v_readlane, so no step goes through LDS.  The result
// is wave-uniform and bit-identical on every lane.  Callers must be converged.
template <int CTRL>
__device__ __forceinline__ float mx_dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float mx_readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

#define MX_DPP_XOR1 0xB1       // quad_perm [1,0,3,2]
#define MX_DPP_XOR2 0x4E       // quad_perm [2,3,0,1]
#define MX_DPP_HALF_MIRROR 0x141
#define MX_DPP_MIRROR 0x140

__device__ __forceinline__ float mx_wave_sum(float v) {
  v += mx_dpp<MX_DPP_XOR1>(v);
  v += mx_dpp<MX_DPP_XOR2>(v);
  v += mx_dpp<MX_DPP_HALF_MIRROR>(v);
  v += mx_dpp<MX_DPP_MIRROR>(v);
  return (mx_readlane(v, 0) + mx_readlane(v, 16)) + (mx_readlane(v, 32) + mx_readlane(v, 48));
}

__device__ __forceinline__ float mx_wave_max(float v) {
  v = fmaxf(v, mx_dpp<MX_DPP_XOR1>(v));
  v = fmaxf(v, mx_dpp<MX_DPP_XOR2>(v));
  v = fmaxf(v, mx_dpp<MX_DPP_HALF_MIRROR>(v));
  v = fmaxf(v, mx_dpp<MX_DPP_MIRROR>(v));
  return fmaxf(fmaxf(mx_readlane(v, 0), mx_readlane(v, 16)),
               fmaxf(mx_readlane(v, 32), mx_readlane(v, 48)));
}

// Reference silu: x / (1 + exp(-x))  (_common.py:83-84).
__device__ __forceinline__ float mx_silu(float x) { return x / (1.0f + expf(-x)); }

// Reference sigmoid: 1 / (1 + exp(-x))  (qwen3_next.py:31-32).
__device__ __forceinline__ float mx_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// fp32 -> fp16 for the intermediates the expert kernels keep in fp16 (activation rows,
// prefill y rows): values beyond the fp16 range saturate to +-65504 instead of becoming
// infinities; NaN stays NaN (both comparisons are false).
__device__ __forceinline__ half_t mx_f16_sat(float v) {
  v = v > 65504.0f ? 65504.0f : v;
  v = v < -65504.0f ? -65504.0f : v;
  return (half_t)v;
}

static inline int mx_ceil_div(int a, int b) { return (a + b - 1) / b; }
static inline size_t mx_align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
