// Elementwise and reduction helpers of the model's producer ops (RMSNorm,
// residual add, SwiGLU) shared by the producer kernels (fused.hip) and the
// M == 1 linears that run a producer inside their x staging (gemv.hip).  Both
// use these same definitions, with the same 8-element chunk per thread and
// the same reduction order, so a fused launch is bit-identical to the pair of
// launches it replaces.
#pragma once

#include "common.hpp"

namespace cider {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ uint16_t lo16(int32_t w) { return (uint16_t)((uint32_t)w & 0xffffu); }
__device__ __forceinline__ uint16_t hi16(int32_t w) { return (uint16_t)((uint32_t)w >> 16); }
__device__ __forceinline__ int32_t pack2(uint16_t a, uint16_t b) {
  return (int32_t)((uint32_t)a | ((uint32_t)b << 16));
}

// h(a + b) elementwise on 8 fp16 values
__device__ __forceinline__ i32x4 add8(i32x4 a, i32x4 b) {
  i32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    r[j] = pack2(f2h(h2f(lo16(a[j])) + h2f(lo16(b[j]))), f2h(h2f(hi16(a[j])) + h2f(hi16(b[j]))));
  return r;
}

__device__ __forceinline__ float sumsq8(i32x4 v, float s) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = h2f(lo16(v[j])), b = h2f(hi16(v[j]));
    s = s + a * a;
    s = s + b * b;
  }
  return s;
}

// RMSNorm output of one element: h(f32(w) * f32(h(x * r)))
__device__ __forceinline__ uint16_t norm1(uint16_t x, uint16_t w, float r) {
  return f2h(h2f(w) * h2f(f2h(h2f(x) * r)));
}

__device__ __forceinline__ i32x4 norm8(i32x4 v, i32x4 w, float r) {
  i32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = pack2(norm1(lo16(v[j]), lo16(w[j]), r), norm1(hi16(v[j]), hi16(w[j]), r));
  return o;
}

// SwiGLU of one element: h(f32(h(silu(g))) * f32(u)), silu(g) = g / (1 + e^-g)
// in fp32 from the hardware exp2 (v_exp_f32, 2^x) and reciprocal
// (v_rcp_f32), each within about one ulp of binary32: the fp32 silu lands
// within a few ulps of the exact quotient, so its fp16 rounding h(silu(g))
// is the exact one or a neighbour only for values within those few ulps of
// a rounding boundary.  (The correctly rounded expf and division took about
// 30 VALU operations per element and bound the SwiGLU kernels.)  Infinities
// map as in the exact expression: g = -inf gives NaN, +inf gives +inf, and
// e^-g overflowing to +inf gives a signed zero.
__device__ __forceinline__ uint16_t swiglu1(uint16_t g, uint16_t u) {
  const float gf = h2f(g);
  constexpr float kLog2e = 1.4426950408889634f;  // 1 / ln 2
  const float e = __builtin_amdgcn_exp2f(-gf * kLog2e);
  const uint16_t a = f2h(gf * __builtin_amdgcn_rcpf(1.0f + e));
  return f2h(h2f(a) * h2f(u));
}

__device__ __forceinline__ i32x4 swiglu8(i32x4 g, i32x4 u) {
  i32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = pack2(swiglu1(lo16(g[j]), lo16(u[j])), swiglu1(hi16(g[j]), hi16(u[j])));
  return o;
}

__device__ __forceinline__ float block_sum4(float v, float* red) {
  const int wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();  // red may still be read from the previous reduction
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

}  // namespace cider
