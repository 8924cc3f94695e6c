// M == 1 decode MV, streaming layout: fp16 activation x int8 weight, no
// activation quantization (the reference's M == 1 semantics,
// cider/kernels/w8a8_int8_mv.metal:14-71 per-channel,
// cider/kernels/pergroup_int8_mv.metal:22-106 per-group):
//   per-channel: y[n] = h(f32(sw[n] * sum_k w[n,k] x[k]) + f32(bias[n]))
//   per-group:   y[n] = h(f32(sum_k f32(sw[k/gs, n] * (w[n,k] x[k])) + bias[n]))
// The reference sums each row across 32 SIMD lanes with Metal's simd_sum,
// whose tree is unspecified; this kernel sums in its own fixed order (below),
// so its fp16 outputs agree with the reference's within fp32 reassociation
// error (the parity bar of the MV tests), not bit for bit.
//
// MI355X layout.  The weight matrix is one HBM stream: a wave owns R
// consecutive rows (R * K contiguous bytes) and lane l loads the 16-byte
// chunks l, l + 64, ..., l + 64 (C - 1) of that range, so every wave
// instruction reads 1 KB of consecutive bytes and a lane's whole share
// (C * 16 bytes) is requested at kernel entry, before x is staged.  R and C
// are compile-time (R * K = 1024 * C), so a chunk's row and column are
// constants plus the lane id.  x is staged once per workgroup in LDS as
// fp16 (2 bytes of LDS read per weight byte).
//
// Arithmetic per 4 weight bytes: one xor maps the signed bytes to b + 128,
// two v_perm_b32 place them under the fp16 exponent of 1024 (bit pattern
// 0x6400 | byte, the value 1024 + b + 128), two packed fp16 subtractions of
// 1152 give the exact integers b as fp16, and two v_dot2_f32_f16 multiply
// them by x and accumulate in fp32: 1.75 VALU operations per weight element.
// The products are exact (8-bit by 11-bit significands); each lane sums its
// chunks' products in chunk order (per group: each chunk's sum times its
// scale), and the 64 lanes of a row are summed in a fixed tree: pairs, quads,
// 8s and 16s by DPP lane moves, then the four 16-lane rows.
//
// Producer modes (XM) stage x' = RMSNorm(x), RMSNorm(x + add) or SwiGLU in
// the same way as the producer kernels (norm_common.hpp, thread t handling the
// 8-element chunks t, t + 256, ...), so a fused launch is bit-identical to
// the producer launch followed by the plain MV.
#include "common.hpp"
#include "dma_common.hpp"
#include "kernels.hpp"
#include "norm_common.hpp"

namespace cider {

namespace {

constexpr int kWpg = 4;  // waves per workgroup (256 threads: the producers' chunk order)

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Exact fp16 values of the four signed bytes of `w`: (bytes 0, 1) in lo,
// (bytes 2, 3) in hi.
__device__ __forceinline__ void bytes_to_h2(uint32_t w, h2& lo, h2& hi) {
  const uint32_t u = w ^ 0x80808080u;                  // b + 128, as unsigned bytes
  const uint32_t plo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t phi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(h2, plo) - off;              // exact: integers below 2048
  hi = __builtin_bit_cast(h2, phi) - off;
}

// sum of the 16 products of one 16-byte weight chunk and its 16 fp16 x
// values (xa: elements 0..7, xb: 8..15), starting from acc.
__device__ __forceinline__ float dot16(i32x4 wv, i32x4 xa, i32x4 xb, float acc) {
  // x dword 2i holds elements 4i, 4i + 1 and dword 2i + 1 elements 4i + 2,
  // 4i + 3 of weight dword i.  The dwords are taken out as scalars first:
  // bit-casting vector elements in place made the compiler read element 0
  // for every index.
  const uint32_t xd[8] = {(uint32_t)xa.x, (uint32_t)xa.y, (uint32_t)xa.z, (uint32_t)xa.w,
                          (uint32_t)xb.x, (uint32_t)xb.y, (uint32_t)xb.z, (uint32_t)xb.w};
  const uint32_t wd[4] = {(uint32_t)wv.x, (uint32_t)wv.y, (uint32_t)wv.z, (uint32_t)wv.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h2 lo, hi;
    bytes_to_h2(wd[i], lo, hi);
    acc = __builtin_amdgcn_fdot2(lo, __builtin_bit_cast(h2, xd[2 * i]), acc, false);
    acc = __builtin_amdgcn_fdot2(hi, __builtin_bit_cast(h2, xd[2 * i + 1]), acc, false);
  }
  return acc;
}

}  // namespace

// SS (per-group, N % (4 R) == 0, 16-byte aligned scales): the workgroup's
// group scales, 4 R consecutive floats of each group row, are loaded as
// 16-byte vectors with x and staged in LDS, instead of one scalar load per
// weight chunk and lane (a group row per lane group, many cache lines per
// instruction).
template <int R, int C, bool PG, int XM, bool SS = false>
__global__ __launch_bounds__(kWpg * 64) void mv_stream_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const float* __restrict__ sw, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, int N, int gs, MvProducer pp) {
  constexpr int K = 1024 * C / R;
  constexpr int CPR = K / 16;  // 16-byte chunks per row
  static_assert(R * K == 1024 * C && CPR >= 64, "one wave covers whole rows");
  static_assert(!SS || PG, "staged scales are per-group");
  __shared__ __attribute__((aligned(16))) uint16_t xs[K];
  constexpr int WR = kWpg * R;                     // rows of the workgroup
  constexpr int SV = SS ? ((K / 64) * R + 255) / 256 : 1;  // scale vectors per thread (gs >= 64)
  __shared__ __attribute__((aligned(16))) float ssc[SS ? (K / 64) * WR : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = (blockIdx.x * kWpg + wave) * R;

  // ---- x (or the producer's inputs) first: the staging then waits for these
  // loads only, and each chunk's products below wait only for that chunk
  constexpr int nchunk = K / 8;
  constexpr int XR = (nchunk + 255) / 256;
  constexpr bool kNorm = XM == XM_NORM || XM == XM_ADDNORM;
  i32x4 xr[XR], xu[XM == XM_SWIGLU || XM == XM_ADDNORM ? XR : 1], xn[kNorm ? XR : 1];
#pragma unroll
  for (int q = 0; q < XR; ++q) {
    const int e = min(tid + q * 256, nchunk - 1);
    xr[q] = ld16(x + 8 * e);
    if constexpr (XM == XM_SWIGLU) xu[q] = ld16(x + K + 8 * e);
    if constexpr (XM == XM_ADDNORM) xu[q] = ld16(pp.add + 8 * e);
    if constexpr (kNorm) xn[q] = ld16(pp.nw + 8 * e);
  }

  // per-group, staged: the [G][WR] scale block of the workgroup's rows
  f32x4 sv[SV];
  const int nw0 = blockIdx.x * WR;
  if constexpr (SS) {
    const int nv = (K / gs) * R;  // 16-byte vectors: R per group row
#pragma unroll
    for (int q = 0; q < SV; ++q) {
      const int e = min(tid + q * 256, nv - 1);
      sv[q] = *reinterpret_cast<const f32x4*>(sw + (int64_t)(e / R) * N + nw0 + 4 * (e % R));
    }
  }

  // per-row scale (per-channel) and bias of the row lane l < R writes; the
  // loads are unconditional (clamped row; x stands in for a missing bias), as
  // a load under a lane mask makes the compiler wait for every load before it
  const int wrow = min(n0 + min(lane, R - 1), N - 1);
  const float s_row = PG ? 0.0f : sw[wrow];
  const float b_row = h2f(bias ? bias[wrow] : x[0]);

  // ---- the wave's weight chunks (rows past N re-read row N - 1: never stored)
  i32x4 wv[C];
  float sj[PG ? C : 1];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = lane + 64 * j;
    const int r = c / CPR, kc = c - r * CPR;
    const int row = min(n0 + r, N - 1);
    wv[j] = ld16_nt(w + (int64_t)row * K + 16 * kc);  // read once: non-temporal
    if constexpr (PG && !SS) sj[j] = sw[(int64_t)((16 * kc) / gs) * N + row];
  }
  // every load is issued before any arithmetic on x: keeps the scheduler from
  // hoisting the producer math (and its waits) above the weight loads
  __builtin_amdgcn_sched_barrier(0);

  // ---- stage x (or x') as fp16; chunks past the end are copies of the last
#pragma unroll
  for (int q = 0; q < XR; ++q) {
    if constexpr (XM == XM_SWIGLU) xr[q] = swiglu8(xr[q], xu[q]);
    if constexpr (XM == XM_ADDNORM) xr[q] = add8(xr[q], xu[q]);
  }
  if constexpr (kNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < XR; ++q) {
      const int e = tid + q * 256;
      if (e < nchunk) {
        if constexpr (XM == XM_ADDNORM)
          if (blockIdx.x == 0) *reinterpret_cast<i32x4*>(pp.hsum + 8 * e) = xr[q];
        ss = sumsq8(xr[q], ss);
      }
    }
    __shared__ float red[4];
    ss = block_sum4(ss, red);
    const float rn = 1.0f / sqrtf(ss / (float)K + pp.eps);
#pragma unroll
    for (int q = 0; q < XR; ++q) xr[q] = norm8(xr[q], xn[q], rn);
  }
  // Unconditional stores: a thread past the last chunk holds a copy of it and
  // writes the same value to the same place.  (Under a lane mask the compiler
  // moves the x load into the masked block, behind the weight loads, and
  // then waits for all of them.)
#pragma unroll
  for (int q = 0; q < XR; ++q) {
    const int e = min(tid + q * 256, nchunk - 1);
    *reinterpret_cast<i32x4*>(xs + 8 * e) = xr[q];
  }
  if constexpr (SS) {
    const int nv = (K / gs) * R;
#pragma unroll
    for (int q = 0; q < SV; ++q) {
      const int e = min(tid + q * 256, nv - 1);  // a copy of the last vector past the end
      *reinterpret_cast<f32x4*>(ssc + (e / R) * WR + 4 * (e % R)) = sv[q];
    }
  }
  __syncthreads();

  // ---- products, in chunk order per lane; a chunk's row is r_lo or r_lo + 1
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = lane + 64 * j;
    const int r = c / CPR, kc = c - r * CPR;
    const i32x4 xa = *reinterpret_cast<const i32x4*>(xs + 16 * kc);
    const i32x4 xb = *reinterpret_cast<const i32x4*>(xs + 16 * kc + 8);
    float d;
    if constexpr (SS) {
      d = ssc[((16 * kc) / gs) * WR + wave * R + r] * dot16(wv[j], xa, xb, 0.0f);
    } else if constexpr (PG) {
      d = sj[j] * dot16(wv[j], xa, xb, 0.0f);
    } else {
      d = dot16(wv[j], xa, xb, 0.0f);
    }
    const int rlo = (64 * j) / CPR;  // constants once the loop is unrolled
    const int rhi = (64 * j + 63) / CPR;
    acc[rlo] = acc[rlo] + (r == rlo ? d : 0.0f);
    if (rhi != rlo) acc[rhi] = acc[rhi] + (r == rhi ? d : 0.0f);
  }
  // ---- rows: sums over the 64 lanes (pairs, quads, 8s and 16s by DPP lane
  // moves, then the four 16-lane rows)
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum_dpp(acc[r]);
  if (lane < R && n0 + lane < N) {
    float a = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r) a = lane == r ? acc[r] : a;
    float v = PG ? a : s_row * a;
    if (bias) v = v + b_row;
    y[n0 + lane] = f2h(v);
  }
}


// Long rows (per-channel; K from 10240 to 16384, K % 1024 == 0): the k range
// splits over the workgroup's KS waves instead of its rows.  Wave v handles k
// in [v K / KS, (v + 1) K / KS) of all KS rows: it loads and stages only that
// part of x (or of the producer's output), into LDS of its own, so no
// workgroup barrier stands before its first product (the RMSNorm producers
// keep one: their row statistic); the waves' partial row sums meet in LDS at
// the end and are added in wave order.  Lane l's chunks are l, l + 64, ... of
// the wave's KS row slices of K / KS bytes (every wave instruction still reads
// 1 KB of consecutive weight bytes within a row, or two runs at a row
// boundary).  Measured against the one-row-per-wave stream (weights from HBM,
// back-to-back launches): N=2560 K=10240 6.95 -> 6.45 us at KS = 5 (512
// workgroups, two per CU; 6.78 us at KS = 4), N=2048 K=12288 6.66 -> 6.27 us;
// at K = 4096 and 8192 it ran level or slower, and the per-group MV level or
// slower, so those keep the stream above.  Producer modes compute x' exactly
// as the producer kernels: SwiGLU per element; RMSNorm's sum of squares by
// threads 0..255 over the 8-element chunks t, t + 256, ... and the 4-wave
// reduction of norm_common.hpp, then each wave normalizes its own range.
template <int K, int KS, int XM>
__global__ __launch_bounds__(KS * 64) void mv_ksplit_kernel(const uint16_t* __restrict__ x,
                                                            const int8_t* __restrict__ w,
                                                            const float* __restrict__ sw,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ y, int N,
                                                            MvProducer pp) {
  constexpr int KQ = K / KS;        // k of one wave
  constexpr int CPQ = KQ / 16;      // 16-byte weight chunks per row and wave
  constexpr int C = KS * CPQ / 64;  // chunks per lane
  static_assert(KQ * KS == K && KS * CPQ == 64 * C && CPQ >= 64, "whole wave loads");
  static_assert(KS >= 4, "the RMSNorm statistic takes threads 0..255");
  constexpr int XCH = KQ / 8;       // 8-element x chunks of the wave's k range
  constexpr int XR = (XCH + 63) / 64;
  constexpr bool kNorm = XM == XM_NORM || XM == XM_ADDNORM;
  constexpr int NCH = K / 8, XRN = (NCH + 255) / 256;  // the statistic's chunks per thread
  __shared__ __attribute__((aligned(16))) uint16_t xs[KS][KQ];
  __shared__ float part[KS][KS];
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * KS;
  const int e0 = wave * XCH;  // the wave's first 8-element chunk

  // x (the producer's inputs of the wave's range) first, then the RMSNorm
  // statistic's chunks, the per-row operands and every weight chunk (clamped
  // rows past N re-read row N - 1 and are never stored)
  i32x4 xr[XR], xu[XM == XM_SWIGLU || XM == XM_ADDNORM ? XR : 1], xn[kNorm ? XR : 1];
#pragma unroll
  for (int q = 0; q < XR; ++q) {
    const int e = e0 + min(lane + 64 * q, XCH - 1);
    xr[q] = ld16(x + 8 * e);
    if constexpr (XM == XM_SWIGLU) xu[q] = ld16(x + K + 8 * e);
    if constexpr (XM == XM_ADDNORM) xu[q] = ld16(pp.add + 8 * e);
    if constexpr (kNorm) xn[q] = ld16(pp.nw + 8 * e);
  }
  i32x4 sr[kNorm ? XRN : 1], su[XM == XM_ADDNORM ? XRN : 1];
  if constexpr (kNorm) {
#pragma unroll
    for (int q = 0; q < XRN; ++q) {
      const int e = min(min(tid, 255) + 256 * q, NCH - 1);
      sr[q] = ld16(x + 8 * e);
      if constexpr (XM == XM_ADDNORM) su[q] = ld16(pp.add + 8 * e);
    }
  }
  const int wrow = min(n0 + min(lane, KS - 1), N - 1);
  const float s_row = sw[wrow];
  const float b_row = h2f(bias ? bias[wrow] : x[0]);
  i32x4 wv[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = lane + 64 * j;
    const int r = c / CPQ, kc = c - r * CPQ;
    wv[j] = ld16_nt(w + (int64_t)min(n0 + r, N - 1) * K + wave * KQ + 16 * kc);
  }
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (XM == XM_SWIGLU) {
#pragma unroll
    for (int q = 0; q < XR; ++q) xr[q] = swiglu8(xr[q], xu[q]);
  }
  if constexpr (kNorm) {
    // the statistic as the producer kernels take it: thread t's chunks t,
    // t + 256, ... (threads 0..255), then the sum over waves 0..3
    float ss = 0.0f;
    if (tid < 256) {
#pragma unroll
      for (int q = 0; q < XRN; ++q) {
        const int e = tid + 256 * q;
        if (e < NCH) {
          i32x4 h = sr[q];
          if constexpr (XM == XM_ADDNORM) {
            h = add8(h, su[q]);
            if (blockIdx.x == 0) *reinterpret_cast<i32x4*>(pp.hsum + 8 * e) = h;
          }
          ss = sumsq8(h, ss);
        }
      }
    }
    ss = wave_sum(ss);
    if (lane == 0 && wave < 4) red[wave] = ss;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float rn = 1.0f / sqrtf(tot / (float)K + pp.eps);
#pragma unroll
    for (int q = 0; q < XR; ++q) {
      i32x4 h = xr[q];
      if constexpr (XM == XM_ADDNORM) h = add8(h, xu[q]);
      xr[q] = norm8(h, xn[q], rn);
    }
  }
  // the wave's x' range, visible to its own lanes after the fence (copies of
  // the last chunk past the end)
#pragma unroll
  for (int q = 0; q < XR; ++q)
    *reinterpret_cast<i32x4*>(&xs[wave][8 * min(lane + 64 * q, XCH - 1)]) = xr[q];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  float acc[KS];
#pragma unroll
  for (int r = 0; r < KS; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = lane + 64 * j;
    const int r = c / CPQ, kc = c - r * CPQ;
    const i32x4 xa = *reinterpret_cast<const i32x4*>(&xs[wave][16 * kc]);
    const i32x4 xb = *reinterpret_cast<const i32x4*>(&xs[wave][16 * kc + 8]);
    const float d = dot16(wv[j], xa, xb, 0.0f);
    const int rlo = (64 * j) / CPQ, rhi = (64 * j + 63) / CPQ;  // constants once unrolled
    acc[rlo] = acc[rlo] + (r == rlo ? d : 0.0f);
    if (rhi != rlo && rhi < KS) acc[rhi] = acc[rhi] + (r == rhi ? d : 0.0f);
  }
  // the wave's partial row sums (the stream's lane tree), then the rows over
  // the waves in wave order
#pragma unroll
  for (int r = 0; r < KS; ++r) acc[r] = wave_sum_dpp(acc[r]);
  if (lane < KS) {
    float a = acc[0];
#pragma unroll
    for (int r = 1; r < KS; ++r) a = lane == r ? acc[r] : a;
    part[wave][lane] = a;
  }
  __syncthreads();
  if (wave == 0 && lane < KS && n0 + lane < N) {
    float a = part[0][lane];
#pragma unroll
    for (int v = 1; v < KS; ++v) a = a + part[v][lane];
    float o = s_row * a;
    if (bias) o = o + b_row;
    y[n0 + lane] = f2h(o);
  }
}

namespace {

template <int R, int C, bool PG, int XM>
hipError_t run_stream(const uint16_t* x, const int8_t* w, const float* sw,
                      const uint16_t* bias, uint16_t* y, int N, int gs, const MvProducer& pp,
                      hipStream_t s) {
  constexpr int K = 1024 * C / R;
  const int waves = (N + R - 1) / R;
  const dim3 grid((waves + kWpg - 1) / kWpg), block(kWpg * 64);
  if constexpr (PG) {
    // staged where it measured faster (weights from HBM): every gs 64 shape
    // (N=2560 K=10240: 11.6 -> 9.5 us), gs 128 at one row per wave (9.4 ->
    // 8.4 us), gs 256 at one row per wave and K >= 8192 (8.4 -> 7.8 us); at
    // two rows per wave gs 128 / 256 ran 3-5 % slower staged
    const bool stage = gs == 64 || (R == 1 && (gs == 128 || K >= 8192));
    if (stage && N % (kWpg * R) == 0 && ((uintptr_t)sw & 15) == 0) {
      mv_stream_kernel<R, C, PG, XM, true><<<grid, block, 0, s>>>(x, w, sw, bias, y, N, gs, pp);
      return hipGetLastError();
    }
  }
  mv_stream_kernel<R, C, PG, XM><<<grid, block, 0, s>>>(x, w, sw, bias, y, N, gs, pp);
  return hipGetLastError();
}

// (R, C) for K: the fewest rows per wave whose R * K is a whole number of
// 1 KB wave loads, with at least 3 chunks per lane in flight; C <= 16.
template <bool PG, int XM>
hipError_t pick_stream(int K, const uint16_t* x, const int8_t* w, const float* sw,
                       const uint16_t* bias, uint16_t* y, int N, int gs, const MvProducer& pp,
                       hipStream_t s) {
#define CIDER_MV(RR, CC) \
  case 1024 * CC / RR: return run_stream<RR, CC, PG, XM>(x, w, sw, bias, y, N, gs, pp, s)
  switch (K) {
    CIDER_MV(4, 4);   // 1024
    CIDER_MV(4, 5);   // 1280
    CIDER_MV(2, 3);   // 1536
    CIDER_MV(4, 7);   // 1792
    CIDER_MV(2, 4);   // 2048
    CIDER_MV(4, 9);   // 2304
    CIDER_MV(2, 5);   // 2560
    CIDER_MV(4, 11);  // 2816
    CIDER_MV(1, 3);   // 3072
    CIDER_MV(4, 13);  // 3328
    CIDER_MV(2, 7);   // 3584
    CIDER_MV(4, 15);  // 3840
    CIDER_MV(1, 4);   // 4096
    CIDER_MV(2, 9);   // 4608
    CIDER_MV(1, 5);   // 5120
    CIDER_MV(2, 11);  // 5632
    CIDER_MV(1, 6);   // 6144
    CIDER_MV(2, 13);  // 6656
    CIDER_MV(1, 7);   // 7168
    CIDER_MV(2, 15);  // 7680
    CIDER_MV(1, 8);   // 8192
    CIDER_MV(1, 9);   // 9216
    CIDER_MV(1, 10);  // 10240
    CIDER_MV(1, 11);  // 11264
    CIDER_MV(1, 12);  // 12288
    CIDER_MV(1, 13);  // 13312
    CIDER_MV(1, 14);  // 14336
    CIDER_MV(1, 15);  // 15360
    CIDER_MV(1, 16);  // 16384
    default: return hipErrorNotSupported;
  }
#undef CIDER_MV
}

// KS of the k-split MV for K (0: not taken): 4 or 5 waves, whichever leaves
// fewer workgroup slots idle in the last round over the CUs (5 needs
// K % 80 == 0).
int ksplit_ways(int N, int K) {
  if (K < 10240 || K > 16384 || K % 1024 != 0) return 0;
  const int cus = num_cus();
  auto idle = [&](int ks) {
    const int wgs = (N + ks - 1) / ks, rounds = (wgs + cus - 1) / cus;
    return (double)(rounds * cus - wgs) / wgs;
  };
  return (K % 80 == 0 && idle(5) < idle(4)) ? 5 : 4;
}

template <int K, int XM>
hipError_t run_ksplit(int ks, const uint16_t* x, const int8_t* w, const float* sw,
                      const uint16_t* bias, uint16_t* y, int N, const MvProducer& pp,
                      hipStream_t s) {
  if constexpr (K % 80 == 0) {
    if (ks == 5) {
      mv_ksplit_kernel<K, 5, XM><<<(N + 4) / 5, 320, 0, s>>>(x, w, sw, bias, y, N, pp);
      return hipGetLastError();
    }
  }
  mv_ksplit_kernel<K, 4, XM><<<(N + 3) / 4, 256, 0, s>>>(x, w, sw, bias, y, N, pp);
  return hipGetLastError();
}

template <int XM>
hipError_t launch_ksplit(int ks, const uint16_t* x, const int8_t* w, const float* sw,
                         const uint16_t* bias, uint16_t* y, int N, int K, const MvProducer& pp,
                         hipStream_t s) {
  switch (K) {
    case 10240: return run_ksplit<10240, XM>(ks, x, w, sw, bias, y, N, pp, s);
    case 11264: return run_ksplit<11264, XM>(ks, x, w, sw, bias, y, N, pp, s);
    case 12288: return run_ksplit<12288, XM>(ks, x, w, sw, bias, y, N, pp, s);
    case 13312: return run_ksplit<13312, XM>(ks, x, w, sw, bias, y, N, pp, s);
    case 14336: return run_ksplit<14336, XM>(ks, x, w, sw, bias, y, N, pp, s);
    case 15360: return run_ksplit<15360, XM>(ks, x, w, sw, bias, y, N, pp, s);
    case 16384: return run_ksplit<16384, XM>(ks, x, w, sw, bias, y, N, pp, s);
    default: return hipErrorNotSupported;
  }
}

bool stream_k(int K) {
  if (K < 1024 || K > 16384 || K % 256 != 0) return false;
  const int m = K / 256;
  if (m % 4 == 0) return true;             // R = 1 (or 2 / 4 at 2048 / 1024)
  if (m % 2 == 0) return K <= 7680;        // R = 2, C = K / 512 <= 15
  return K <= 3840;                         // R = 4, C = K / 256 <= 15
}

}  // namespace

bool mv_stream_supported(const void* x, const void* w, const void* sw, int K, int gs) {
  return stream_k(K) && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
         (gs == 0 || gs % 16 == 0) && (((uintptr_t)sw & 3) == 0);
}

hipError_t launch_mv_stream(int xm, const uint16_t* x, const int8_t* w, const float* sw,
                            const uint16_t* bias, uint16_t* y, int N, int K, int gs,
                            const MvProducer& pp, hipStream_t s) {
  if (gs > 0) {
    if (xm != XM_PLAIN) return hipErrorInvalidValue;
    return pick_stream<true, XM_PLAIN>(K, x, w, sw, bias, y, N, gs, pp, s);
  }
  // the k-split MV for every producer mode alike, so a fused launch still
  // equals the producer launch followed by the plain MV bit for bit
  if (const int ks = ksplit_ways(N, K)) {
    switch (xm) {
      case XM_PLAIN: return launch_ksplit<XM_PLAIN>(ks, x, w, sw, bias, y, N, K, pp, s);
      case XM_NORM: return launch_ksplit<XM_NORM>(ks, x, w, sw, bias, y, N, K, pp, s);
      case XM_ADDNORM: return launch_ksplit<XM_ADDNORM>(ks, x, w, sw, bias, y, N, K, pp, s);
      case XM_SWIGLU: return launch_ksplit<XM_SWIGLU>(ks, x, w, sw, bias, y, N, K, pp, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (xm) {
    case XM_PLAIN: return pick_stream<false, XM_PLAIN>(K, x, w, sw, bias, y, N, 0, pp, s);
    case XM_NORM: return pick_stream<false, XM_NORM>(K, x, w, sw, bias, y, N, 0, pp, s);
    case XM_ADDNORM: return pick_stream<false, XM_ADDNORM>(K, x, w, sw, bias, y, N, 0, pp, s);
    case XM_SWIGLU: return pick_stream<false, XM_SWIGLU>(K, x, w, sw, bias, y, N, 0, pp, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace cider
