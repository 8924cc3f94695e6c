// Decode-sized int8 GEMV: 1 <= M <= 4 quantized activation rows against int8
// or packed int4 weights, with the library's int32 / per-channel / per-group
// epilogues.  This is the memory-bound kernel for the reference's small-M
// dispatches (cider/kernels/w8a8_matmul.metal:301-453 "_small" variants,
// cider/kernels/pergroup_int8_gemm.metal:198-223 "_small", and W4A8 at every
// M, csrc/src/w4a8_primitive.mm:175-264) when only a handful of tokens is in
// flight.  Same arithmetic as the GEMMs:
//   acc  = sum_k q[m,k] w[n,k]                          exact int32
//   PC   y = h(f32(f32(acc) * sa[m]) * sw[n] (+ bias))
//   PG   y = h(f32(chain * sa[m]) (+ bias)),  chain = (((0 + t_0) + t_1) + ...)
//        t_g = f32(f32(D_g) * sw[g, n]) over the groups in order
//   I32  y = acc
//
// MI355X design: the weight stream is the whole cost, so the kernel reads each
// weight row the way a copy kernel would: one wave per row, lane l takes the
// 16-byte chunks l, l + 64, ... of the row (a wave instruction covers 1 KB of
// one row), and every chunk of the row is requested at kernel entry.  The
// quantized activations (M x K int8, at most 64 KB) are staged in LDS once per
// 16-row workgroup.  Products use v_dot4 (4 int8 MACs into int32, exact); int4
// weights are widened in registers first.  Per-group: the chunks of one group
// sit in consecutive lanes of one instruction, so D_g is a shuffle reduction
// over those lanes (exact); its term goes to LDS, and one lane per activation
// row runs the sequential chain over the groups.
#include "common.hpp"
#include "kernels.hpp"
#include "quant_common.hpp"

namespace cider {

namespace {

constexpr int kRowsPerWg = 16;  // one wave per weight row

__device__ __forceinline__ int dot16(i32x4 w, i32x4 x, int acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_sdot4(w[j], x[j], acc, false);
  return acc;
}

template <bool SWH>
__device__ __forceinline__ float scale1(const void* base, int64_t idx) {
  if constexpr (SWH)
    return h2f(reinterpret_cast<const uint16_t*>(base)[idx]);
  else
    return reinterpret_cast<const float*>(base)[idx];
}

// JM: chunks per lane (row bytes <= 64 * 16 * JM); MT: activation rows.
// FQ: p.x holds the fp16 activations and the workgroup quantizes them per
// token while staging them (bit-identical to quantize_per_token: the same
// absmax, scale and rounding helpers), so no separate quantize launch.
template <int MT, int WF, int EPI, bool SWH, int GS, int JM, bool FQ>
__global__ __launch_bounds__(1024) void gemv_q_kernel(const GemmArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  __shared__ float red[MT][16];
  __shared__ float srow[MT];
  const int M = p.M, N = p.N, K = p.K;
  int8_t* xs = reinterpret_cast<int8_t*>(dyn);  // [MT][K]
  const int G = (EPI == EPI_PG) ? K / GS : 0;
  float* tg = reinterpret_cast<float*>(dyn + (size_t)MT * K);  // [16][MT][GP]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = blockIdx.x * kRowsPerWg + wave;
  const bool live = n < N;
  const int rb = (WF == W_I4) ? K / 2 : K;  // bytes per weight row
  const int nc = rb >> 4;                    // 16-byte chunks per row
  const int8_t* wr = reinterpret_cast<const int8_t*>(p.w) + (int64_t)(live ? n : 0) * rb;

  // ---- the whole row in flight (chunks past the end re-read the last one)
  i32x4 wv[JM];
#pragma unroll
  for (int j = 0; j < JM; ++j) wv[j] = ld16_nt(wr + 16 * min(lane + 64 * j, nc - 1));

  // ---- stage the quantized activations
  if constexpr (FQ) {
    constexpr int QV = 2;  // 8-element vectors per thread and row (K <= 16384)
    const uint16_t* x16 = reinterpret_cast<const uint16_t*>(p.x);
    const int nv8 = K >> 3;
    i32x4 xv[MT][QV];
    float am[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      am[m] = 0.0f;
#pragma unroll
      for (int i = 0; i < QV; ++i) {
        const int e = tid + 1024 * i;
        xv[m][i] = (m < M && e < nv8) ? ld16(x16 + (size_t)m * K + 8 * e) : i32x4{0, 0, 0, 0};
        am[m] = absmax8(xv[m][i], am[m]);
      }
      am[m] = wave_max(am[m]);
      if (lane == 0) red[m][wave] = am[m];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float a = red[m][0];
#pragma unroll
      for (int w = 1; w < 16; ++w) a = fmaxf(a, red[m][w]);
      const float sc = row_scale(a);
      const float inv = 1.0f / sc;
      if (tid == 0) srow[m] = sc;
#pragma unroll
      for (int i = 0; i < QV; ++i) {
        const int e = tid + 1024 * i;
        if (m < M && e < nv8)
          *reinterpret_cast<i32x2*>(xs + (size_t)m * K + 8 * e) = quant8(xv[m][i], inv);
      }
    }
  } else {
    const int xc = (M * K) >> 4;
    for (int e = tid; e < xc; e += 1024)
      *reinterpret_cast<i32x4*>(xs + 16 * e) = ld16(p.x + 16 * e);
  }
  __syncthreads();
  if (!live) return;  // uniform per wave; no barrier follows

  int acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0;
  constexpr int CPG = (EPI == EPI_PG) ? (WF == W_I4 ? GS / 32 : GS / 16) : 1;  // chunks per group
  const int GP = (G + 3) & ~3;  // padded row of terms (16-byte aligned)
  float* tw = tg + (size_t)wave * MT * GP;

#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int c = lane + 64 * j;
    if (64 * j >= nc) break;  // uniform
    const bool in = c < nc;
    int d[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) d[m] = 0;
    if (in) {
      if constexpr (WF == W_I4) {
        // 16 bytes = 32 int4 = k 32c .. 32c + 31, low nibble first
        i32x4 lo, hi;
        uint32_t a0, a1;
        unpack_w4_word((uint32_t)wv[j][0], a0, a1);
        lo[0] = (int)a0;
        lo[1] = (int)a1;
        unpack_w4_word((uint32_t)wv[j][1], a0, a1);
        lo[2] = (int)a0;
        lo[3] = (int)a1;
        unpack_w4_word((uint32_t)wv[j][2], a0, a1);
        hi[0] = (int)a0;
        hi[1] = (int)a1;
        unpack_w4_word((uint32_t)wv[j][3], a0, a1);
        hi[2] = (int)a0;
        hi[3] = (int)a1;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m >= M) break;
          const int8_t* xp = xs + (size_t)m * K + 32 * c;
          d[m] = dot16(lo, *reinterpret_cast<const i32x4*>(xp), d[m]);
          d[m] = dot16(hi, *reinterpret_cast<const i32x4*>(xp + 16), d[m]);
        }
      } else {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m >= M) break;
          d[m] = dot16(wv[j], *reinterpret_cast<const i32x4*>(xs + (size_t)m * K + 16 * c), d[m]);
        }
      }
    }
    if constexpr (EPI == EPI_PG) {
      // D_g over the CPG consecutive lanes of each group (exact int32)
#pragma unroll
      for (int m = 0; m < MT; ++m) d[m] = group_sum_i32<CPG>(d[m]);
      if (in && (lane % CPG) == 0) {
        const int g = c / CPG;
        const float sw = scale1<SWH>(p.sw, (int64_t)g * N + n);
#pragma unroll
        for (int m = 0; m < MT; ++m) tw[m * GP + g] = (float)d[m] * sw;
      }
    } else {
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[m] += d[m];
    }
  }

  if constexpr (EPI == EPI_PG) {
    // the wave's own LDS slice: writes by other lanes of this wave are visible
    // after the wave-level fence
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < MT && lane < M) {
      const int m = lane;
      const float* tm = tw + m * GP;
      float chain = 0.0f;
      int g = 0;
      for (; g + 8 <= G; g += 8) {  // eight terms read ahead of their adds
        const f32x4 a = *reinterpret_cast<const f32x4*>(tm + g);
        const f32x4 b = *reinterpret_cast<const f32x4*>(tm + g + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) chain = chain + a[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) chain = chain + b[i];
      }
      for (; g < G; ++g) chain = chain + tm[g];
      float v = chain * (FQ ? srow[m] : p.sa[m]);
      if (p.bias) v = v + h2f(p.bias[n]);
      reinterpret_cast<uint16_t*>(p.y)[(int64_t)m * N + n] = f2h(v);
    }
  } else {
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = wave_sum_i32(acc[m]);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m >= M) break;
        if constexpr (EPI == EPI_I32) {
          reinterpret_cast<int32_t*>(p.y)[(int64_t)m * N + n] = acc[m];
        } else {
          float v = (float)acc[m] * (FQ ? srow[m] : p.sa[m]);
          v = v * reinterpret_cast<const float*>(p.sw)[n];
          if (p.bias) v = v + h2f(p.bias[n]);
          reinterpret_cast<uint16_t*>(p.y)[(int64_t)m * N + n] = f2h(v);
        }
      }
    }
  }
}

template <int MT, int WF, int EPI, bool SWH, int GS, bool FQ>
hipError_t run_jm(const GemmArgs& a, hipStream_t s) {
  const int rb = (WF == W_I4) ? a.K / 2 : a.K;
  const int per_lane = (rb / 16 + 63) / 64;
  const int GP = (EPI == EPI_PG) ? ((a.K / GS + 3) & ~3) : 0;
  const size_t lds = (size_t)MT * a.K + (size_t)kRowsPerWg * MT * GP * sizeof(float);
  const dim3 grid((a.N + kRowsPerWg - 1) / kRowsPerWg), block(64 * kRowsPerWg);
#define CIDER_GQ(J) gemv_q_kernel<MT, WF, EPI, SWH, GS, J, FQ><<<grid, block, lds, s>>>(a)
  if (per_lane <= 2)
    CIDER_GQ(2);
  else if (per_lane <= 3)
    CIDER_GQ(3);
  else if (per_lane <= 4)
    CIDER_GQ(4);
  else if (per_lane <= 6)
    CIDER_GQ(6);
  else if (per_lane <= 8)
    CIDER_GQ(8);
  else if (per_lane <= 12)
    CIDER_GQ(12);
  else if constexpr (!(FQ && MT == 4))  // 16 chunks + 4 staged x rows: no room
    CIDER_GQ(16);
  else
    return hipErrorInvalidValue;
#undef CIDER_GQ
  return hipGetLastError();
}

template <int MT, bool FQ>
hipError_t run_mt(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s) {
  if (epi == EPI_I32) return run_jm<MT, W_I8, EPI_I32, false, 0, FQ>(a, s);
  if (epi == EPI_PC) {
    if (wf == W_I4) return run_jm<MT, W_I4, EPI_PC, false, 0, FQ>(a, s);
    return run_jm<MT, W_I8, EPI_PC, false, 0, FQ>(a, s);
  }
  if (wf == W_I4) {  // int4 per-group scales are fp16
    if (gs == 64) return run_jm<MT, W_I4, EPI_PG, true, 64, FQ>(a, s);
    return run_jm<MT, W_I4, EPI_PG, true, 128, FQ>(a, s);
  }
  if (gs == 64) return run_jm<MT, W_I8, EPI_PG, false, 64, FQ>(a, s);
  if (gs == 128) return run_jm<MT, W_I8, EPI_PG, false, 128, FQ>(a, s);
  return run_jm<MT, W_I8, EPI_PG, false, 256, FQ>(a, s);
}

template <bool FQ>
hipError_t run_m(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s) {
  switch (a.M) {
    case 1: return run_mt<1, FQ>(a, wf, epi, gs, s);
    case 2: return run_mt<2, FQ>(a, wf, epi, gs, s);
    default: return run_mt<4, FQ>(a, wf, epi, gs, s);
  }
}


// ---- M == 1, int4 weights, per-group fp16 or per-channel fp32 scales, x
// quantized in the kernel:
// the streaming layout of the decode MV (mv_stream.hip) instead of one wave
// per row.  A wave owns R consecutive weight rows (R * K / 2 contiguous
// bytes) and lane l requests the 16-byte chunks l, l + 64, ..., l + 64 (C - 1)
// of them at entry, so each lane has C loads in flight (the one-row waves
// above have K / 2048, two at K = 4096).  Each workgroup quantizes x (the
// quantize kernel's helpers: the same q and scale) into LDS and stages the
// fp16 group scales of its NW * R rows as 16-byte vectors.  A chunk is 32 k of
// one row and one group (gs 64 / 128), the CPG chunks of a group sit in
// consecutive lanes: D_g is their shuffle sum (exact int32), its term
// f32(f32(D_g) * s) goes to LDS, and one lane per row chains the terms in
// group order, then y = h(f32(chain * sa) (+ bias)), as the kernel above.
// Per-channel (GS == 0): each lane sums its chunks per row (exact int32), the
// rows' sums meet in xor butterflies, y = h(f32(f32(acc) * sa) * sw[n] (+ bias)).
template <int R, int C, int GS, int NW>
__global__ __launch_bounds__(64 * NW) void gemv1_w4_kernel(const uint16_t* __restrict__ x16,
                                                          const uint8_t* __restrict__ w,
                                                          const void* __restrict__ sw_,
                                                          const uint16_t* __restrict__ bias,
                                                          uint16_t* __restrict__ y, int N) {
  constexpr bool PG = GS > 0;
  constexpr int NT = 64 * NW;
  constexpr int RB = 1024 * C / R, K = 2 * RB;  // bytes per weight row, k per row
  constexpr int CPR = RB / 16, CPG = PG ? GS / 32 : 1, G = PG ? K / GS : 1;
  constexpr int WR = NW * R;                      // weight rows of the workgroup
  constexpr int NV8 = K / 8, XV = (NV8 + NT - 1) / NT;
  constexpr int SVN = PG ? G * WR / 8 : 1, SV = PG ? (SVN + NT - 1) / NT : 1;  // scale vectors
  static_assert(R * RB == 1024 * C && CPR % CPG == 0 && 64 % CPG == 0, "chunk layout");
  static_assert(WR % 8 == 0, "whole 16-byte scale vectors per group row");
  const uint16_t* sw = reinterpret_cast<const uint16_t*>(sw_);
  __shared__ __attribute__((aligned(16))) int8_t xq[K];
  __shared__ __attribute__((aligned(16))) uint16_t ssc[PG ? G * WR : 8];
  __shared__ __attribute__((aligned(16))) float terms[NW][R][PG ? G : 1];
  __shared__ float red[NW];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw0 = blockIdx.x * WR, n0 = nw0 + wave * R;

  // x, the scale block and every weight chunk requested first (clamped, so
  // the loads are unconditional; rows past N are never stored)
  i32x4 xv[XV];
#pragma unroll
  for (int q = 0; q < XV; ++q) xv[q] = ld16(x16 + 8 * min(tid + NT * q, NV8 - 1));
  i32x4 sv[SV];
  if constexpr (PG) {
#pragma unroll
    for (int q = 0; q < SV; ++q) {
      const int e = min(tid + NT * q, SVN - 1);
      const int g = e / (WR / 8), part = e % (WR / 8);
      sv[q] = ld16(sw + (int64_t)g * N + min(nw0 + 8 * part, N - 8));
    }
  }
  i32x4 wv[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = lane + 64 * j, r = c / CPR, kc = c % CPR;
    wv[j] = ld16_nt(w + (int64_t)min(n0 + r, N - 1) * RB + 16 * kc);
  }
  __builtin_amdgcn_sched_barrier(0);

  // per-token quantization of x (one row)
  float am = 0.0f;
#pragma unroll
  for (int q = 0; q < XV; ++q)
    if (tid + NT * q < NV8) am = absmax8(xv[q], am);
  am = wave_max(am);
  if (lane == 0) red[wave] = am;
  if constexpr (PG) {
#pragma unroll
    for (int q = 0; q < SV; ++q) {
      const int e = tid + NT * q;
      if (e < SVN) *reinterpret_cast<i32x4*>(ssc + 8 * e) = sv[q];
    }
  }
  __syncthreads();
  float a = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) a = fmaxf(a, red[i]);
  const float sa = row_scale(a), inv = 1.0f / sa;
#pragma unroll
  for (int q = 0; q < XV; ++q) {
    const int e = tid + NT * q;
    if (e < NV8) *reinterpret_cast<i32x2*>(xq + 8 * e) = quant8(xv[q], inv);
  }
  __syncthreads();

  // chunks: 32 int4 (k 32 kc .. 32 kc + 31, low nibble first) against 32 q
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = lane + 64 * j, r = c / CPR, kc = c % CPR;
    i32x4 lo, hi;
    uint32_t a0, a1;
    unpack_w4_word((uint32_t)wv[j][0], a0, a1);
    lo[0] = (int)a0;
    lo[1] = (int)a1;
    unpack_w4_word((uint32_t)wv[j][1], a0, a1);
    lo[2] = (int)a0;
    lo[3] = (int)a1;
    unpack_w4_word((uint32_t)wv[j][2], a0, a1);
    hi[0] = (int)a0;
    hi[1] = (int)a1;
    unpack_w4_word((uint32_t)wv[j][3], a0, a1);
    hi[2] = (int)a0;
    hi[3] = (int)a1;
    int d = dot16(lo, *reinterpret_cast<const i32x4*>(xq + 32 * kc), 0);
    d = dot16(hi, *reinterpret_cast<const i32x4*>(xq + 32 * kc + 16), d);
    if constexpr (PG) {
      d = group_sum_i32<CPG>(d);
      if ((lane % CPG) == 0) {
        const int g = kc / CPG;
        terms[wave][r][g] = (float)d * h2f(ssc[g * WR + wave * R + r]);
      }
    } else {
      // the chunk's row is rlo or rlo + 1 (constants once unrolled)
      const int rlo = (64 * j) / CPR, rhi = (64 * j + 63) / CPR;
      acc[rlo] += r == rlo ? d : 0;
      if (rhi != rlo && rhi < R) acc[rhi] += r == rhi ? d : 0;
    }
  }
  if constexpr (!PG) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[r] = wave_sum_i32(acc[r]);
    if (lane < R && n0 + lane < N) {
      int av = acc[0];
#pragma unroll
      for (int r = 1; r < R; ++r) av = lane == r ? acc[r] : av;
      float v = (float)av * sa;
      v = v * reinterpret_cast<const float*>(sw_)[n0 + lane];
      if (bias) v = v + h2f(bias[n0 + lane]);
      y[n0 + lane] = f2h(v);
    }
    return;
  }
  // the wave's own LDS slice: visible to its other lanes after the fence
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < R && n0 + lane < N) {
    const float* tm = terms[wave][lane];
    float chain = 0.0f;
#pragma unroll 8
    for (int g = 0; g < G; ++g) chain = chain + tm[g];
    float v = chain * sa;
    if (bias) v = v + h2f(bias[n0 + lane]);
    y[n0 + lane] = f2h(v);
  }
}

// (R, C, NW) of the streaming M == 1 kernel for K: four 4-row waves up to
// K = 8192, eight 1-row waves above (whole 1 KB wave loads need R * K / 2 to
// be a multiple of 1024).  Measured against the one-row-per-wave kernel, fused
// quantization in both, weights from HBM: N=12288 K=4096 gs 128 10.4 -> 7.9
// us, gs 64 10.8 -> 8.1 us; N=4096 K=12288 gs 128 11.1 -> 9.6 us, gs 64 11.9
// -> 11.0 us; per-channel N=12288 K=4096 9.3 -> 7.4 us, N=4096 K=12288 9.2 ->
// 8.0 us.
template <int GS>
hipError_t run_gemv1_w4(const uint16_t* x, const GemmArgs& a, hipStream_t s) {
  const uint8_t* w = reinterpret_cast<const uint8_t*>(a.w);
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
#define CIDER_G1(RR, CC, NWW)                                                                 \
  case 1024 * (CC) / (RR) * 2:                                                                \
    gemv1_w4_kernel<RR, CC, GS, NWW><<<(a.N + (NWW) * (RR) - 1) / ((NWW) * (RR)), 64 * (NWW), \
                                       0, s>>>(x, w, a.sw, a.bias, y, a.N);                   \
    return hipGetLastError();
  switch (a.K) {
    CIDER_G1(4, 4, 4)   // 2048
    CIDER_G1(4, 6, 4)   // 3072
    CIDER_G1(4, 8, 4)   // 4096
    CIDER_G1(4, 10, 4)  // 5120
    CIDER_G1(4, 12, 4)  // 6144
    CIDER_G1(4, 14, 4)  // 7168
    CIDER_G1(4, 16, 4)  // 8192
    CIDER_G1(1, 5, 8)   // 10240
    CIDER_G1(1, 6, 8)   // 12288
    CIDER_G1(1, 7, 8)   // 14336
    CIDER_G1(1, 8, 8)   // 16384
    default: return hipErrorNotSupported;
  }
#undef CIDER_G1
}

bool gemv1_w4_supported(const GemmArgs& a, int wf, int epi, int gs) {
  return a.M == 1 && wf == W_I4 && (epi == EPI_PC || (epi == EPI_PG && (gs == 64 || gs == 128))) &&
         a.K >= 2048 && a.K <= 16384 && a.K % 1024 == 0 && (a.K <= 8192 || a.K % 2048 == 0) &&
         a.N % 8 == 0 && ((uintptr_t)a.w & 15) == 0 && ((uintptr_t)a.sw & 15) == 0;
}

}  // namespace

bool gemv_q_supported(const GemmArgs& a, int wf, bool fused) {
  const int rb = (wf == W_I4) ? a.K / 2 : a.K;
  const int per_lane = (rb / 16 + 63) / 64;
  return a.M >= 1 && a.M <= 4 && a.K <= 16384 && a.K % (wf == W_I4 ? 32 : 16) == 0 &&
         !(fused && a.M > 2 && per_lane > 12) && ((uintptr_t)a.x & 15) == 0 &&
         ((uintptr_t)a.w & 15) == 0;
}

hipError_t launch_gemv_q(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s) {
  return run_m<false>(a, wf, epi, gs, s);
}

hipError_t launch_gemv_qx(const uint16_t* x, const GemmArgs& a, int wf, int epi, int gs,
                          hipStream_t s) {
  if (gemv1_w4_supported(a, wf, epi, gs) && ((uintptr_t)x & 15) == 0) {
    if (epi == EPI_PC) return run_gemv1_w4<0>(x, a, s);
    return gs == 64 ? run_gemv1_w4<64>(x, a, s) : run_gemv1_w4<128>(x, a, s);
  }
  GemmArgs b = a;
  b.x = reinterpret_cast<const int8_t*>(x);
  b.sa = nullptr;
  return run_m<true>(b, wf, epi, gs, s);
}

}  // namespace cider
