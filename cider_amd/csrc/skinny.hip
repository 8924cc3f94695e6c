// Skinny int8 GEMM for small M (2 <= M <= 64, and W4A8 at M == 1): the
// regime where the weight stream from HBM, not the MFMA rate, sets the time.
//
// Same epilogues as the tiled kernel (gemm.hip), same reference semantics:
//   EPI_I32 cider/kernels/w8a8_matmul.metal:301-453 (the reference's "_small"
//           variant for M <= 64, csrc/src/w8a8_primitive.mm:295-330)
//   EPI_PC  cider/kernels/w8a8_matmul.metal:63-81, :280-295
//   EPI_PG  cider/kernels/pergroup_int8_gemm.metal:152-189
//
// MI355X design
//   * A workgroup (4 waves) owns 16 weight rows n and all M (<= 16*TM) rows
//     of x.  The four waves split K into contiguous ranges; every lane loads
//     its weight slice straight from HBM into the MFMA "A" register (no LDS
//     round trip: each weight byte is used by TM MFMAs only).  Two register
//     buffers of U k-steps alternate, so the next batch is in flight while
//     the current one reduces.
//   * Per-group scales of the workgroup's 16 columns (all groups) are staged
//     in LDS at the start; their loads are issued before the first weight
//     batch, so the flush never waits on a global load inside the loop.
//   * Per-channel / int32: the four int32 partial accumulators are summed
//     through LDS (exact, order-free) and wave 0 runs the epilogue.
//   * Per-group: each wave flushes its groups into an fp32 chain in group
//     order; the four chains are then added in wave order.  The int32 group
//     sums are exact; the fp32 association differs from a single sequential
//     chain by at most an fp32 rounding (far below one fp16 ulp).
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

constexpr int kThreads = 256;

template <bool SWH>
__device__ __forceinline__ float load_scale1(const void* base, int64_t idx) {
  if constexpr (SWH)
    return h2f(reinterpret_cast<const uint16_t*>(base)[idx]);
  else
    return reinterpret_cast<const float*>(base)[idx];
}

}  // namespace

template <int TM, int WF, int EPI, bool SWH, int GS, bool VEC>
__global__ __launch_bounds__(kThreads) void skinny_kernel(const GemmArgs p) {
  constexpr int U = (TM == 1) ? 8 : 4;                 // k-steps per batch
  constexpr int SUB = (EPI == EPI_PG) ? GS / 64 : 1;   // k-steps per group
  constexpr int SR = 8;                                // scale loads per thread in registers
  __shared__ __attribute__((aligned(16))) int32_t red[4][TM][kWave][4];
  // per-group scales of this workgroup's 16 columns, [group][column] in fp32
  extern __shared__ __attribute__((aligned(16))) float ssc[];

  // The wave index must be a scalar: branches on k (group start / end) then
  // stay uniform.  MFMA ignores EXEC, so an MFMA under a divergent branch
  // would execute in both arms.
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 15, lq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int n0 = blockIdx.x * 16;
  const int nw = n0 + lrow;  // weight row this lane loads
  const int8_t* __restrict__ X = p.x;
  const int8_t* __restrict__ W = reinterpret_cast<const int8_t*>(p.w);
  const int64_t ldw = (WF == W_I4) ? (K >> 1) : K;

  const int nkb = (K + 63) / 64;  // 64-wide k steps
  const int ngrp = (nkb + SUB - 1) / SUB;
  const int gper = (ngrp + 3) / 4;
  const int kb0 = min(wave * gper * SUB, nkb);
  const int kb1 = min((wave + 1) * gper * SUB, nkb);

  // ---- per-group scales: requested first, so the LDS stores below wait
  // only for them while the first weight batch is already in flight
  const int G = (EPI == EPI_PG) ? K / GS : 0;
  float sr[SR];
  auto load_sc = [&](int e) -> float {
    const int g = e >> 4, c = e & 15;
    return (n0 + c < N) ? load_scale1<SWH>(p.sw, (int64_t)g * N + n0 + c) : 0.0f;
  };
  if constexpr (EPI == EPI_PG) {
#pragma unroll
    for (int q = 0; q < SR; ++q) {
      const int e = tid + q * kThreads;
      if (e < G * 16) sr[q] = load_sc(e);
    }
  }

  // one batch of U k-steps starting at kb: weight fragments and x fragments
  auto load_batch = [&](int kb, i32x4 (&wv)[U], i32x4 (&xv)[U][TM]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = kb + u;
      const bool in = k < kb1;
      // weight slice: k elements [64k + 16lq, +16) of row nw
      if constexpr (WF == W_I4) {
        const int byte = k * 32 + 8 * lq;
        const int nb = (in && nw < N) ? (int)ldw - byte : 0;
        i32x4 raw;
        if (nb <= 0)
          raw = i32x4{0, 0, 0, 0};
        else if (VEC)
          { const i32x2 v = ld8(W + (int64_t)nw * ldw + byte); raw = i32x4{v[0], v[1], 0, 0}; }
        else
          raw = load_bytes_partial(W + (int64_t)nw * ldw + byte, nb < 8 ? nb : 8);
        wv[u] = raw;  // unpacked at consumption
      } else {
        const int kk = k * 64 + 16 * lq;
        const int nb = (in && nw < N) ? K - kk : 0;
        if (nb <= 0)
          wv[u] = i32x4{0, 0, 0, 0};
        else if (VEC)
          wv[u] = ld16(W + (int64_t)nw * K + kk);
        else
          wv[u] = load_bytes_partial(W + (int64_t)nw * K + kk, nb < 16 ? nb : 16);
      }
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int m = b * 16 + lrow;
        const int kk = k * 64 + 16 * lq;
        const int nb = (in && m < M) ? K - kk : 0;
        if (nb <= 0)
          xv[u][b] = i32x4{0, 0, 0, 0};
        else if (VEC)
          xv[u][b] = ld16(X + (int64_t)m * K + kk);
        else
          xv[u][b] = load_bytes_partial(X + (int64_t)m * K + kk, nb < 16 ? nb : 16);
      }
    }
  };

  i32x4 acc[TM];
  float facc[TM][4];
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    acc[b] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < 4; ++r) facc[b][r] = 0.0f;
  }
  const int ncol = n0 + 4 * lq;  // first output column of this lane

  auto consume = [&](int kb, const i32x4 (&wv)[U], const i32x4 (&xv)[U][TM]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = kb + u;
      if (k >= kb1) break;  // uniform
      i32x4 wf = wv[u];
      if constexpr (WF == W_I4) {
        uint32_t o0, o1, o2, o3;
        unpack_w4_word((uint32_t)wv[u][0], o0, o1);
        unpack_w4_word((uint32_t)wv[u][1], o2, o3);
        wf = i32x4{(int)o0, (int)o1, (int)o2, (int)o3};
      }
      if constexpr (EPI == EPI_PG) {
        const bool first = (k % SUB) == 0, last = (k % SUB) == SUB - 1;
        if (first) {
#pragma unroll
          for (int b = 0; b < TM; ++b) acc[b] = mfma_i8(wf, xv[u][b], i32x4{0, 0, 0, 0});
        } else {
#pragma unroll
          for (int b = 0; b < TM; ++b) acc[b] = mfma_i8(wf, xv[u][b], acc[b]);
        }
        if (last) {
          const f32x4 swv = *reinterpret_cast<const f32x4*>(&ssc[(k / SUB) * 16 + 4 * lq]);
#pragma unroll
          for (int b = 0; b < TM; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float t = (float)acc[b][r] * swv[r];
              facc[b][r] = facc[b][r] + t;
            }
        }
      } else {
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[b] = mfma_i8(wf, xv[u][b], acc[b]);
      }
    }
  };

  // ---- two register buffers: the next batch loads while this one reduces
  i32x4 wa[U], xa[U][TM], wb[U], xb[U][TM];
  load_batch(kb0, wa, xa);
  if constexpr (EPI == EPI_PG) {
#pragma unroll
    for (int q = 0; q < SR; ++q) {
      const int e = tid + q * kThreads;
      if (e < G * 16) ssc[e] = sr[q];
    }
    for (int e = tid + SR * kThreads; e < G * 16; e += kThreads) ssc[e] = load_sc(e);
    __syncthreads();
  }
  for (int kb = kb0; kb < kb1; kb += 2 * U) {
    if (kb + U < kb1) load_batch(kb + U, wb, xb);
    consume(kb, wa, xa);
    if (kb + U >= kb1) break;
    if (kb + 2 * U < kb1) load_batch(kb + 2 * U, wa, xa);
    consume(kb + U, wb, xb);
  }

  // ---- combine the four K ranges
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    if constexpr (EPI == EPI_PG) {
      *reinterpret_cast<f32x4*>(&red[wave][b][lane][0]) =
          f32x4{facc[b][0], facc[b][1], facc[b][2], facc[b][3]};
    } else {
      *reinterpret_cast<i32x4*>(&red[wave][b][lane][0]) = acc[b];
    }
  }
  __syncthreads();
  if (wave != 0) return;

#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int m = b * 16 + lrow;
    if constexpr (EPI == EPI_PG) {
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(&red[w][b][lane][0]);
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[b][r] = facc[b][r] + v[r];
      }
    } else {
#pragma unroll
      for (int w = 1; w < 4; ++w) acc[b] += *reinterpret_cast<const i32x4*>(&red[w][b][lane][0]);
    }
    if (m >= M || ncol >= N) continue;
    if constexpr (EPI == EPI_I32) {
      int32_t* yp = reinterpret_cast<int32_t*>(p.y) + (int64_t)m * N + ncol;
      if (VEC) {
        *reinterpret_cast<i32x4*>(yp) = acc[b];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (ncol + r < N) yp[r] = acc[b][r];
      }
    } else {
      const float sam = p.sa[m];
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = ncol + r;
        float v;
        if constexpr (EPI == EPI_PC) {
          const float swn = n < N ? reinterpret_cast<const float*>(p.sw)[n] : 0.0f;
          v = (float)acc[b][r] * sam;
          v = v * swn;
        } else {
          v = facc[b][r] * sam;
        }
        if (p.bias) v = v + (n < N ? h2f(p.bias[n]) : 0.0f);
        o[r] = f2h(v);
      }
      uint16_t* yp = reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + ncol;
      if (VEC) {
        *reinterpret_cast<i32x2*>(yp) =
            i32x2{(int)(o[0] | ((uint32_t)o[1] << 16)), (int)(o[2] | ((uint32_t)o[3] << 16))};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (ncol + r < N) yp[r] = o[r];
      }
    }
  }
}

namespace {

template <int TM, int WF, int EPI, bool SWH, int GS>
hipError_t run_skinny(const GemmArgs& a, bool vec, hipStream_t s) {
  const int grid = (a.N + 15) / 16;
  // per-group: the workgroup's 16 columns of every group's scales in LDS
  const size_t lds = (EPI == EPI_PG) ? (size_t)(a.K / GS) * 16 * sizeof(float) : 0;
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  if (vec)
    skinny_kernel<TM, WF, EPI, SWH, GS, true><<<grid, kThreads, lds, s>>>(a);
  else
    skinny_kernel<TM, WF, EPI, SWH, GS, false><<<grid, kThreads, lds, s>>>(a);
  return hipGetLastError();
}

template <int TM>
hipError_t dispatch_tm(const GemmArgs& a, int wf, int epi, bool sw_half, int gs,
                       bool vec, hipStream_t s) {
  if (epi == EPI_I32) return run_skinny<TM, W_I8, EPI_I32, false, 0>(a, vec, s);
  if (epi == EPI_PC) {
    if (wf == W_I4) return run_skinny<TM, W_I4, EPI_PC, false, 0>(a, vec, s);
    return run_skinny<TM, W_I8, EPI_PC, false, 0>(a, vec, s);
  }
  if (wf == W_I4) {
    (void)sw_half;  // int4 per-group scales are fp16
    if (gs == 64) return run_skinny<TM, W_I4, EPI_PG, true, 64>(a, vec, s);
    return run_skinny<TM, W_I4, EPI_PG, true, 128>(a, vec, s);
  }
  if (gs == 64) return run_skinny<TM, W_I8, EPI_PG, false, 64>(a, vec, s);
  if (gs == 128) return run_skinny<TM, W_I8, EPI_PG, false, 128>(a, vec, s);
  return run_skinny<TM, W_I8, EPI_PG, false, 256>(a, vec, s);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

hipError_t launch_skinny(const GemmArgs& a, int wf, int epi, bool sw_half,
                         int gs, hipStream_t s) {
  const bool vec = (wf == W_I4 ? a.K % 32 == 0 : a.K % 16 == 0) && a.N % 4 == 0 &&
                   aligned16(a.x) && aligned16(a.w) && aligned16(a.y);
  if (a.M <= 16) return dispatch_tm<1>(a, wf, epi, sw_half, gs, vec, s);
  if (a.M <= 32) return dispatch_tm<2>(a, wf, epi, sw_half, gs, vec, s);
  return dispatch_tm<4>(a, wf, epi, sw_half, gs, vec, s);
}

}  // namespace cider
