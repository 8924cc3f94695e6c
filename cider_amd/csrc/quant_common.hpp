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

// amax over a 256-thread workgroup (4 waves); red: 4 floats of LDS.  Every
// thread gets the result.
__device__ __forceinline__ float block_max4(float v, float* red) {
  const int wave = threadIdx.x >> 6;
  v = wave_max(v);
  __syncthreads();  // red may still be read from the previous reduction
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float row_scale(float amax) {
  float s = amax / 127.0f;
  return s == 0.0f ? 1.0f : s;
}

// q of one element x (an fp16 value widened to binary32):
//   * r = x * inv rounded to binary32, as a fused multiply-add with +0: the
//     exact product rounded once, as the multiply rounds it (the two differ
//     only in the sign of a zero product, which q does not see), and the
//     fp16 -> fp32 widening folds into v_fma_mix_f32;
//   * clamped to [-128, 127] first (fmax(NaN, -128) = -128): rounding and
//     clamping commute here, since the bounds are integers;
//   * rounded half away from zero as the truncation of r + copysign(0.5 -
//     2^-25, r): adding the largest float below 0.5 carries r past the next
//     integer exactly when its fraction is >= 0.5 (checked against roundf for
//     every binary32 value), and the conversion to int truncates.
__device__ __forceinline__ int32_t quant1i(float xv, float inv) {
  float r = __builtin_fmaf(xv, inv, 0.0f);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  r = r + __builtin_copysignf(0x1.fffffep-2f, r);
  return (int32_t)r;
}

__device__ __forceinline__ int8_t quant1(float xv, float inv) {
  return (int8_t)quant1i(xv, inv);
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
    const uint32_t a = (uint32_t)quant1i(h2f((uint16_t)(w & 0xffffu)), inv) & 0xffu;
    const uint32_t b = (uint32_t)quant1i(h2f((uint16_t)(w >> 16)), inv) & 0xffu;
    const uint32_t pair = a | (b << 8);
    if (j & 1)
      out[j >> 1] |= pair << 16;
    else
      out[j >> 1] = pair;
  }
  return i32x2{(int32_t)out[0], (int32_t)out[1]};
}

}  // namespace cider
