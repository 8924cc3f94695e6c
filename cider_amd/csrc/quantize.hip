// Per-token activation quantization (fp16 [M,K] -> int8 [M,K] + fp32 [M]).
//
// Semantics of cider/kernels/w8a8_quantize.metal:33-86:
//   amax = max_k |x[m,k]|        (fmax: NaN never wins)
//   s    = amax / 127, s == 0 -> 1
//   inv  = 1 / s
//   q    = clamp(round_half_away(x * inv), -128, 127)   (NaN -> -128)
//
// MI355X design: one 64-lane wavefront owns one row, so the absmax is a pure
// cross-lane reduction (no LDS, no barrier); a workgroup of 4 waves handles 4
// rows.  Up to 64 rows (decode-sized batches) get a 1024-thread workgroup per
// row instead, and rows of 2048 to 16384 elements a 256-thread one, except
// at M >= 2048 with rows of at most 3072 elements.  A row stays in registers between the absmax and the quantize pass
// (each element is read from HBM once); rows past 16384 elements are re-read,
// which hits in L2.
#include "common.hpp"
#include "kernels.hpp"
#include "quant_common.hpp"

namespace cider {

// Vectorized rows: K % 8 == 0, x 16-byte and q 8-byte aligned.  NV > 0 keeps
// NV 16-byte vectors per lane in registers; NV == 0 streams the row twice.
template <int NV>
__global__ __launch_bounds__(256) void quantize_vec_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q,
    float* __restrict__ sa, int M, int K) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;  // uniform per wave
  const uint16_t* xr = x + row * K;
  int8_t* qr = q + row * K;
  const int nvec = K >> 3;
  float amax = 0.0f;
  if constexpr (NV > 0) {
    // every load first, unconditional (clamped: a lane past the row re-reads
    // its last vector, which leaves the max unchanged), as a load under a
    // lane mask makes the compiler wait for each before the next: M=4096
    // K=2560 5.99 -> 5.79 us, M=2048 K=4096 5.37 -> 4.98 us (M=8192 level)
    i32x4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = ld16(xr + 8 * min(lane + i * kWave, nvec - 1));
#pragma unroll
    for (int i = 0; i < NV; ++i) amax = absmax8(v[i], amax);
    amax = wave_max(amax);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (lane == 0) sa[row] = s;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + i * kWave;
      if (e < nvec) *reinterpret_cast<i32x2*>(qr + 8 * e) = quant8(v[i], inv);
    }
  } else {
    for (int e = lane; e < nvec; e += kWave) amax = absmax8(ld16(xr + 8 * e), amax);
    amax = wave_max(amax);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (lane == 0) sa[row] = s;
    for (int e = lane; e < nvec; e += kWave)
      *reinterpret_cast<i32x2*>(qr + 8 * e) = quant8(ld16(xr + 8 * e), inv);
  }
}

// A workgroup of NT threads per row: few rows (M <= 64, NT = 1024: sixteen
// waves share a row's loads and conversions, where a single wave per row
// leaves the row's VALU work serial: about 8 us at K = 12288) and long rows
// (NT = 256); the absmax goes through LDS in wave order.  Vectorized rows
// only; NV 16-byte vectors per thread.
template <int NV, int NT = 1024>
__global__ __launch_bounds__(NT) void quantize_row_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q,
    float* __restrict__ sa, int K) {
  constexpr int NWV = NT / 64;
  __shared__ float red[NWV];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * K;
  int8_t* qr = q + row * K;
  const int nvec = K >> 3;
  i32x4 v[NV];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + i * NT;
    v[i] = e < nvec ? ld16(xr + 8 * e) : i32x4{0, 0, 0, 0};
    amax = absmax8(v[i], amax);
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < NWV; ++w) amax = fmaxf(amax, red[w]);
  const float s = row_scale(amax);
  const float inv = 1.0f / s;
  if (tid == 0) sa[row] = s;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = tid + i * NT;
    if (e < nvec) *reinterpret_cast<i32x2*>(qr + 8 * e) = quant8(v[i], inv);
  }
}

// Any K and alignment: element-wise, two passes.
__global__ __launch_bounds__(256) void quantize_scalar_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q,
    float* __restrict__ sa, int M, int K) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* xr = x + row * K;
  int8_t* qr = q + row * K;
  float amax = 0.0f;
  for (int k = lane; k < K; k += kWave) amax = fmaxf(amax, fabsf(h2f(xr[k])));
  amax = wave_max(amax);
  const float s = row_scale(amax);
  const float inv = 1.0f / s;
  if (lane == 0) sa[row] = s;
  for (int k = lane; k < K; k += kWave) qr[k] = quant1(h2f(xr[k]), inv);
}

hipError_t launch_quantize(const uint16_t* x, int8_t* q, float* sa, int M,
                           int K, hipStream_t s) {
  const dim3 grid((M + 3) / 4), block(256);
  const bool vec = (K % 8 == 0) && (((uintptr_t)x & 15) == 0) &&
                   (((uintptr_t)q & 7) == 0);
  if (!vec) {
    quantize_scalar_kernel<<<grid, block, 0, s>>>(x, q, sa, M, K);
    return hipGetLastError();
  }
  const int nvec = K >> 3;
  if (M <= 64 && nvec > 64 && nvec <= 8 * 1024) {
    // a row per 1024-thread workgroup (max(a, b) is exact, so the absmax does
    // not depend on how the row is split)
    if (nvec <= 1024)
      quantize_row_kernel<1><<<M, 1024, 0, s>>>(x, q, sa, K);
    else if (nvec <= 2048)
      quantize_row_kernel<2><<<M, 1024, 0, s>>>(x, q, sa, K);
    else if (nvec <= 4096)
      quantize_row_kernel<4><<<M, 1024, 0, s>>>(x, q, sa, K);
    else
      quantize_row_kernel<8><<<M, 1024, 0, s>>>(x, q, sa, K);
    return hipGetLastError();
  }
  const int per_lane = (nvec + kWave - 1) / kWave;
  // Many rows of up to 3072 elements: one wave per row, the row in at most 6
  // vectors per lane (4096 x 2560: 7.5 -> 6.4 us, 8192 x 2560: 13.0 -> 11.4
  // us, 4096 x 2048: 6.8 -> 5.4 us against the 256-thread row workgroups;
  // level at M <= 1024).
  const bool wave_rows = M >= 2048 && per_lane <= 6;
  if (!wave_rows && nvec >= 256 && nvec <= 8 * 256) {
    // Rows of 2048 .. 16384 elements at any M: a 256-thread workgroup per
    // row, its four waves' maxima meeting in LDS.  One wave per row held up
    // to 32 16-byte vectors per lane and ran at few waves per SIMD (4096 x
    // 10240: 36.3 -> 21.7 us; 4096 x 4096: 10.8 -> 9.7 us).
    const int nv = (nvec + 255) / 256;
    if (nv <= 2) quantize_row_kernel<2, 256><<<M, 256, 0, s>>>(x, q, sa, K);
    else if (nv <= 3) quantize_row_kernel<3, 256><<<M, 256, 0, s>>>(x, q, sa, K);
    else if (nv <= 4) quantize_row_kernel<4, 256><<<M, 256, 0, s>>>(x, q, sa, K);
    else if (nv <= 5) quantize_row_kernel<5, 256><<<M, 256, 0, s>>>(x, q, sa, K);
    else if (nv <= 6) quantize_row_kernel<6, 256><<<M, 256, 0, s>>>(x, q, sa, K);
    else quantize_row_kernel<8, 256><<<M, 256, 0, s>>>(x, q, sa, K);
    return hipGetLastError();
  }
  if (per_lane <= 1)
    quantize_vec_kernel<1><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else if (per_lane <= 2)
    quantize_vec_kernel<2><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else if (per_lane <= 4)
    quantize_vec_kernel<4><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else if (per_lane <= 5)
    quantize_vec_kernel<5><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else if (per_lane <= 6)
    quantize_vec_kernel<6><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else if (per_lane <= 8)
    quantize_vec_kernel<8><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else if (per_lane <= 16)
    quantize_vec_kernel<16><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else if (per_lane <= 32)
    quantize_vec_kernel<32><<<grid, block, 0, s>>>(x, q, sa, M, K);
  else
    quantize_vec_kernel<0><<<grid, block, 0, s>>>(x, q, sa, M, K);
  return hipGetLastError();
}

}  // namespace cider
