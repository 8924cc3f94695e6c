// Device helpers of the per-token quantization (cider/kernels/w8a8_quantize.metal:33-86),
// shared by the quantize kernel and the producer kernels that end in it.
//   amax = max_k |x[m,k]|        (fmax: NaN never wins)
//   s    = amax / 127, s == 0 -> 1
//   inv  = 1 / s
//   q    = clamp(round_half_away(x * inv), -128, 127)   (NaN -> -128)
#pragma once

#include "common.hpp"

namespace cider {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float row_scale(float amax) {
  float s = amax / 127.0f;
  return s == 0.0f ? 1.0f : s;
}

__device__ __forceinline__ int8_t quant1(float xv, float inv) {
  float r = __builtin_roundf(xv * inv);  // half away from zero
  r = fminf(fmaxf(r, -128.0f), 127.0f);  // fmax(NaN, -128) = -128
  return (int8_t)(int)r;
}

__device__ __forceinline__ float absmax8(i32x4 v, float m) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = (uint32_t)v[j];
    m = fmaxf(m, fabsf(h2f((uint16_t)(w & 0xffffu))));
    m = fmaxf(m, fabsf(h2f((uint16_t)(w >> 16))));
  }
  return m;
}

__device__ __forceinline__ i32x2 quant8(i32x4 v, float inv) {
  uint32_t out[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = (uint32_t)v[j];
    const uint32_t a = (uint8_t)quant1(h2f((uint16_t)(w & 0xffffu)), inv);
    const uint32_t b = (uint8_t)quant1(h2f((uint16_t)(w >> 16)), inv);
    const uint32_t pair = a | (b << 8);
    if (j & 1)
      out[j >> 1] |= pair << 16;
    else
      out[j >> 1] = pair;
  }
  return i32x2{(int32_t)out[0], (int32_t)out[1]};
}

}  // namespace cider
