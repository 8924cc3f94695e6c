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
  for (int j = 0; j < JM; ++j) wv[j] = ld16(wr + 16 * min(lane + 64 * j, nc - 1));

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
      for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int off = CPG / 2; off >= 1; off >>= 1) d[m] += __shfl_xor(d[m], off);
      }
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
    for (int m = 0; m < MT; ++m) {
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off);
    }
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
  GemmArgs b = a;
  b.x = reinterpret_cast<const int8_t*>(x);
  b.sa = nullptr;
  return run_m<true>(b, wf, epi, gs, s);
}

}  // namespace cider
