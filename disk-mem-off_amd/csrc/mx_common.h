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

__device__ __forceinline__ float mx_wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, MX_WAVE);
  return v;
}

__device__ __forceinline__ float mx_wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, MX_WAVE));
  return v;
}

// Reference silu: x / (1 + exp(-x))  (_common.py:83-84).
__device__ __forceinline__ float mx_silu(float x) { return x / (1.0f + expf(-x)); }

// Reference sigmoid: 1 / (1 + exp(-x))  (qwen3_next.py:31-32).
__device__ __forceinline__ float mx_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

static inline int mx_ceil_div(int a, int b) { return (a + b - 1) / b; }
static inline size_t mx_align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
