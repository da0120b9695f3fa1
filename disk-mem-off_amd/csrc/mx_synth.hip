// Synthetic weights and offline per-row int8 quantisation on the device.
//
// mx_fill_normal is the device twin of moe_mi355x/gen.py: element i of stream
// (seed, stream_id) is
//   key = mix(mix(seed) ^ (stream_id * 0xD1B54A32D192ED03))
//   x0 = mix(key + (2 c) * G), x1 = mix(key + (2 c + 1) * G),   c = offset + i
//   u1 = ((x0 >> 11) + 1) * 2^-53,  u2 = (x1 >> 11) * 2^-53
//   z = sqrt(-2 ln u1) * cos(2 pi u2)          (fp64, Box-Muller)
//   value = fp32(std * z)   [then fp16(value) for fp16 output]
// with mix the SplitMix64 finaliser and G = 0x9E3779B97F4A7C15.
//
// mx_quantize_rows_i8 implements the per-output-channel symmetric int8 scheme, the
// zero-point-0 / per-row-scale case of the reference formula (q - zp) * scale
// (offload_runtime/quantize.py:44).
#include <math.h>

#include "mx_common.h"

__device__ __forceinline__ uint64_t mx_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename T>
__global__ __launch_bounds__(256) void k_fill_normal(T* __restrict__ dst, size_t n, uint64_t key,
                                                     uint64_t offset, double stdv) {
  const uint64_t G = 0x9E3779B97F4A7C15ull;
  const double two53 = 1.0 / 9007199254740992.0;  // 2^-53
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint64_t c = offset + i;
    const uint64_t x0 = mx_mix64(key + (2ull * c) * G);
    const uint64_t x1 = mx_mix64(key + (2ull * c + 1ull) * G);
    const double u1 = (double)((x0 >> 11) + 1ull) * two53;
    const double u2 = (double)(x1 >> 11) * two53;
    const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    const float v = (float)(stdv * z);
    dst[i] = (T)v;
  }
}

extern "C" int mx_fill_normal(void* dst, int32_t dtype, size_t n, uint64_t seed, uint64_t stream_id,
                              uint64_t offset, float std, void* stream) {
  if (!dst && n) return MX_ERR_INVALID;
  if (n == 0) return MX_OK;
  // Host copy of mx_mix64 for the key.
  auto mix = [](uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  };
  const uint64_t key = mix(mix(seed) ^ (stream_id * 0xD1B54A32D192ED03ull));
  const size_t blocks_needed = (n + 255) / 256;
  const unsigned blocks = (unsigned)(blocks_needed < 65536 ? blocks_needed : 65536);
  mx_clear_error();
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MX_DT_F32)
    hipLaunchKernelGGL(k_fill_normal<float>, dim3(blocks), dim3(256), 0, s, (float*)dst, n, key,
                       offset, (double)std);
  else if (dtype == MX_DT_F16)
    hipLaunchKernelGGL(k_fill_normal<half_t>, dim3(blocks), dim3(256), 0, s, (half_t*)dst, n, key,
                       offset, (double)std);
  else
    return MX_ERR_INVALID;
  return mx_launch_status();
}

// One 256-thread block per row.
template <typename T>
__global__ __launch_bounds__(256) void k_quantize_rows(const T* __restrict__ w, int cols,
                                                       int8_t* __restrict__ q,
                                                       half_t* __restrict__ scale) {
  const int r = blockIdx.x;
  const T* wr = w + (size_t)r * cols;
  float amax = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) amax = fmaxf(amax, fabsf((float)wr[c]));
  __shared__ float red[4];
  amax = mx_wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  half_t sh = (half_t)(amax / 127.0f);
  if (amax == 0.f || (float)sh == 0.f) sh = (half_t)1.0f;
  const float s = (float)sh;
  if (threadIdx.x == 0) scale[r] = sh;
  int8_t* qr = q + (size_t)r * cols;
  for (int c = threadIdx.x; c < cols; c += 256) {
    float v = rintf((float)wr[c] / s);
    v = fminf(127.f, fmaxf(-127.f, v));
    qr[c] = (int8_t)(int)v;
  }
}

extern "C" int mx_quantize_rows_i8(const void* w, int32_t w_dtype, int32_t rows, int32_t cols,
                                   int8_t* q, void* scale, void* stream) {
  if (!w || !q || !scale || rows < 0 || cols <= 0) return MX_ERR_INVALID;
  if (rows == 0) return MX_OK;
  mx_clear_error();
  hipStream_t s = (hipStream_t)stream;
  if (w_dtype == MX_DT_F32)
    hipLaunchKernelGGL(k_quantize_rows<float>, dim3(rows), dim3(256), 0, s, (const float*)w,
                       (int)cols, q, (half_t*)scale);
  else if (w_dtype == MX_DT_F16)
    hipLaunchKernelGGL(k_quantize_rows<half_t>, dim3(rows), dim3(256), 0, s, (const half_t*)w,
                       (int)cols, q, (half_t*)scale);
  else
    return MX_ERR_INVALID;
  return mx_launch_status();
}
