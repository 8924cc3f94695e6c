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
//   * A workgroup (KW = 4, 8 or 16 waves) owns 16 weight rows n and all M
//     (<= 16*TM) rows of x.  The waves split K into contiguous ranges (more
//     waves when N alone gives the grid too few to keep HBM busy); every lane loads
//     its weight slice straight from HBM into the MFMA "A" register (no LDS
//     round trip: each weight byte is used by TM MFMAs only).  Two register
//     buffers of U k-steps alternate, so the next batch is in flight while
//     the current one reduces.
//   * Per-group scales of the workgroup's 16 columns (all groups) are staged
//     in LDS at the start; their loads are issued before the first weight
//     batch, so the flush never waits on a global load inside the loop.
//   * Per-channel / int32: the KW int32 partial accumulators are summed
//     through LDS (exact, order-free) and wave 0 runs the epilogue.
//   * Per-group keeps the reference's single sequential fp32 chain over the
//     groups: skinny_pg_kernel below, which deals the groups to the waves
//     round-robin instead of in contiguous K ranges.
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

template <bool SWH>
__device__ __forceinline__ float load_scale1(const void* base, int64_t idx) {
  if constexpr (SWH)
    return h2f(reinterpret_cast<const uint16_t*>(base)[idx]);
  else
    return reinterpret_cast<const float*>(base)[idx];
}

}  // namespace

template <int TM, int WF, int EPI, bool SWH, int GS, bool VEC, int KW>
__global__ __launch_bounds__(KW * 64) void skinny_kernel(const GemmArgs p) {
  // k-steps per batch: two batches in flight per lane; 16-wave workgroups
  // have 128 VGPRs per lane, which holds two batches of 6 (int4) or 4 (int8)
  constexpr int U = (TM == 1) ? (KW == 16 ? (WF == W_I4 ? 6 : 4) : 8) : 4;
  static_assert(EPI != EPI_PG, "per-group runs skinny_pg_kernel");
  __shared__ __attribute__((aligned(16))) int32_t red[KW][TM][kWave][4];

  // The wave index must be a scalar: branches on k stay uniform.  MFMA
  // ignores EXEC, so an MFMA under a divergent branch would execute in both
  // arms.
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
  const int kper = (nkb + KW - 1) / KW;
  const int kb0 = min(wave * kper, nkb);
  const int kb1 = min((wave + 1) * kper, nkb);

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
          wv[u] = ld16_nt(W + (int64_t)nw * K + kk);
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
#pragma unroll
  for (int b = 0; b < TM; ++b) acc[b] = i32x4{0, 0, 0, 0};
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
#pragma unroll
      for (int b = 0; b < TM; ++b) acc[b] = mfma_i8(wf, xv[u][b], acc[b]);
    }
  };

  // ---- two register buffers: the next batch loads while this one reduces
  i32x4 wa[U], xa[U][TM], wb[U], xb[U][TM];
  load_batch(kb0, wa, xa);
  for (int kb = kb0; kb < kb1; kb += 2 * U) {
    if (kb + U < kb1) load_batch(kb + U, wb, xb);
    consume(kb, wa, xa);
    if (kb + U >= kb1) break;
    if (kb + 2 * U < kb1) load_batch(kb + 2 * U, wa, xa);
    consume(kb + U, wb, xb);
  }

  // ---- combine the KW K ranges (int32: exact in any order)
#pragma unroll
  for (int b = 0; b < TM; ++b) *reinterpret_cast<i32x4*>(&red[wave][b][lane][0]) = acc[b];
  __syncthreads();
  if (wave != 0) return;

#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int m = b * 16 + lrow;
#pragma unroll
    for (int w = 1; w < KW; ++w) acc[b] += *reinterpret_cast<const i32x4*>(&red[w][b][lane][0]);
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
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = ncol + r;
        const float swn = n < N ? reinterpret_cast<const float*>(p.sw)[n] : 0.0f;
        v[r] = (float)acc[b][r] * sam;
        v[r] = v[r] * swn;
        if (p.bias) v[r] = v[r] + (n < N ? h2f(p.bias[n]) : 0.0f);
      }
      const uint32_t o01 = f2h2(v[0], v[1]), o23 = f2h2(v[2], v[3]);
      uint16_t* yp = reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + ncol;
      if (VEC) {
        *reinterpret_cast<i32x2*>(yp) = i32x2{(int)o01, (int)o23};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (ncol + r < N) yp[r] = (uint16_t)((r < 2 ? o01 : o23) >> (16 * (r & 1)));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Per-group, M <= 64, in the reference's order: one fp32 chain per output over
// the groups in sequence (cider/kernels/pergroup_int8_gemm.metal:152-189).
// The KW waves take the groups round-robin (wave w: groups w, w + KW, ...), so
// a round of KW consecutive groups completes together: each wave writes its
// group's terms t = f32(D_g) * sw[g, n] for the workgroup's outputs into an LDS
// slice, and after the round's barrier the owner of each output adds the KW
// terms in group order.  Weights and x are prefetched across rounds (two
// register batches of RB rounds), so the barriers do not drain the stream.
// ---------------------------------------------------------------------------
template <int TM, int WF, bool SWH, int GS, bool VEC, int KW>
__global__ __launch_bounds__(KW * 64) void skinny_pg_kernel(const GemmArgs p) {
  constexpr int kThreads = KW * 64;
  constexpr int SUB = GS / 64;  // k-steps per group
  constexpr int UK = (TM == 1) ? (KW == 16 ? (WF == W_I4 ? 6 : 4) : 8) : 4;
  constexpr int RB = UK / SUB > 0 ? UK / SUB : 1;  // rounds per batch
  constexpr int U = RB * SUB;                       // k-steps per batch
  constexpr int SR = 8;
  constexpr int NOUT = TM * 256;                    // outputs of the workgroup
  constexpr int OWN = (NOUT + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) float tb[2][KW][NOUT];
  extern __shared__ __attribute__((aligned(16))) float ssc[];  // [G][16] scales

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 15, lq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int n0 = blockIdx.x * 16;
  const int nw = n0 + lrow;
  const int8_t* __restrict__ X = p.x;
  const int8_t* __restrict__ W = reinterpret_cast<const int8_t*>(p.w);
  const int64_t ldw = (WF == W_I4) ? (K >> 1) : K;
  const int G = K / GS;
  const int R = (G + KW - 1) / KW;  // rounds (the same for every wave)
  const int nks = R * SUB;          // k-steps per wave, padding rounds included

  float sr[SR];
  auto load_sc = [&](int e) -> float {
    const int g = e >> 4, c = e & 15;
    return (n0 + c < N) ? load_scale1<SWH>(p.sw, (int64_t)g * N + n0 + c) : 0.0f;
  };
#pragma unroll
  for (int q = 0; q < SR; ++q) {
    const int e = tid + q * kThreads;
    if (e < G * 16) sr[q] = load_sc(e);
  }

  // k-step i of this wave: step i % SUB of group wave + KW * (i / SUB); rounds
  // past the last group re-load the last group (their terms are not used)
  auto load_batch = [&](int i0, i32x4 (&wv)[U], i32x4 (&xv)[U][TM]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = min(i0 + u, nks - 1);
      const int k = min(wave + KW * (i / SUB), G - 1) * SUB + i % SUB;
      if constexpr (WF == W_I4) {
        const int byte = k * 32 + 8 * lq;
        if (nw >= N)
          wv[u] = i32x4{0, 0, 0, 0};
        else if (VEC)
          { const i32x2 v = ld8(W + (int64_t)nw * ldw + byte); wv[u] = i32x4{v[0], v[1], 0, 0}; }
        else
          wv[u] = load_bytes_partial(W + (int64_t)nw * ldw + byte, 8);
      } else {
        const int kk = k * 64 + 16 * lq;
        if (nw >= N)
          wv[u] = i32x4{0, 0, 0, 0};
        else if (VEC)
          wv[u] = ld16_nt(W + (int64_t)nw * K + kk);
        else
          wv[u] = load_bytes_partial(W + (int64_t)nw * K + kk, 16);
      }
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int m = b * 16 + lrow;
        const int kk = k * 64 + 16 * lq;
        if (m >= M)
          xv[u][b] = i32x4{0, 0, 0, 0};
        else if (VEC)
          xv[u][b] = ld16(X + (int64_t)m * K + kk);
        else
          xv[u][b] = load_bytes_partial(X + (int64_t)m * K + kk, 16);
      }
    }
  };

  float facc[OWN];
#pragma unroll
  for (int o = 0; o < OWN; ++o) facc[o] = 0.0f;

  auto consume = [&](int i0, const i32x4 (&wv)[U], const i32x4 (&xv)[U][TM]) {
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      const int r = i0 / SUB + rr;
      if (r >= R) break;  // uniform: every wave has R rounds
      i32x4 d[TM];
#pragma unroll
      for (int s = 0; s < SUB; ++s) {
        const int u = rr * SUB + s;
        i32x4 wf = wv[u];
        if constexpr (WF == W_I4) {
          uint32_t o0, o1, o2, o3;
          unpack_w4_word((uint32_t)wv[u][0], o0, o1);
          unpack_w4_word((uint32_t)wv[u][1], o2, o3);
          wf = i32x4{(int)o0, (int)o1, (int)o2, (int)o3};
        }
#pragma unroll
        for (int b = 0; b < TM; ++b)
          d[b] = mfma_i8(wf, xv[u][b], s == 0 ? i32x4{0, 0, 0, 0} : d[b]);
      }
      const int g = wave + KW * r;
      const f32x4 swv = *reinterpret_cast<const f32x4*>(&ssc[min(g, G - 1) * 16 + 4 * lq]);
      float* slot = &tb[r & 1][wave][0];
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        f32x4 t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = (float)d[b][e] * swv[e];
        *reinterpret_cast<f32x4*>(slot + b * 256 + lane * 4) = t;
      }
      __syncthreads();
      const int nv = min(KW, G - r * KW);  // groups of this round, in order
#pragma unroll
      for (int o = 0; o < OWN; ++o) {
        const int idx = tid + o * kThreads;
        if (idx < NOUT)
          for (int w = 0; w < nv; ++w) facc[o] = facc[o] + tb[r & 1][w][idx];
      }
    }
  };

  i32x4 wa[U], xa[U][TM], wb[U], xb[U][TM];
  load_batch(0, wa, xa);
#pragma unroll
  for (int q = 0; q < SR; ++q) {
    const int e = tid + q * kThreads;
    if (e < G * 16) ssc[e] = sr[q];
  }
  for (int e = tid + SR * kThreads; e < G * 16; e += kThreads) ssc[e] = load_sc(e);
  __syncthreads();
  for (int i0 = 0; i0 < nks; i0 += 2 * U) {
    if (i0 + U < nks) load_batch(i0 + U, wb, xb);
    consume(i0, wa, xa);
    if (i0 + U >= nks) break;
    if (i0 + 2 * U < nks) load_batch(i0 + 2 * U, wa, xa);
    consume(i0 + U, wb, xb);
  }

  // ---- epilogue: output idx = (b, lane, e) of the MFMA layout: weight row
  // n0 + 4 * (lane / 16) + e, activation row 16 b + lane % 16
#pragma unroll
  for (int o = 0; o < OWN; ++o) {
    const int idx = tid + o * kThreads;
    if (idx >= NOUT) continue;
    const int b = idx >> 8, l = (idx >> 2) & 63, e = idx & 3;
    const int n = n0 + 4 * (l >> 4) + e, m = b * 16 + (l & 15);
    if (m >= M || n >= N) continue;
    float v = facc[o] * p.sa[m];
    if (p.bias) v = v + h2f(p.bias[n]);
    reinterpret_cast<uint16_t*>(p.y)[(int64_t)m * N + n] = f2h(v);
  }
}

namespace {

template <int TM, int WF, int EPI, bool SWH, int GS, int KW>
hipError_t run_skinny_kw(const GemmArgs& a, bool vec, size_t lds, hipStream_t s) {
  const int grid = (a.N + 15) / 16;
  if (vec)
    skinny_kernel<TM, WF, EPI, SWH, GS, true, KW><<<grid, KW * 64, lds, s>>>(a);
  else
    skinny_kernel<TM, WF, EPI, SWH, GS, false, KW><<<grid, KW * 64, lds, s>>>(a);
  return hipGetLastError();
}

template <int TM, int WF, bool SWH, int GS, int KW>
hipError_t run_skinny_pg_kw(const GemmArgs& a, bool vec, size_t lds, hipStream_t s) {
  const int grid = (a.N + 15) / 16;
  if (vec)
    skinny_pg_kernel<TM, WF, SWH, GS, true, KW><<<grid, KW * 64, lds, s>>>(a);
  else
    skinny_pg_kernel<TM, WF, SWH, GS, false, KW><<<grid, KW * 64, lds, s>>>(a);
  return hipGetLastError();
}

// Waves per workgroup: 4, raised to 8 or 16 while the grid has fewer than 16
// waves per CU and every wave keeps at least 4 k-steps of its own (per-group:
// two rounds of groups).  The LDS slices (KW x TM x 1 KB per buffer) cap KW at
// 16 for TM = 1 and 8 for TM = 2 and 4.  At TM = 4 a lane holds ~200 VGPRs,
// so an 8-wave workgroup fills a CU: 8 waves only while the grid is one round
// of workgroups (N=4096 K=12288 M=33, per-group int8 gs 64: 60.0 vs 39.4 us,
// per-channel int4: 23.7 vs 21.8 us; at N=6144, 384 workgroups, 4 waves stay
// faster: 19.0 vs 23.6 us per-group, 15.6 vs 17.5 us per-channel).
template <int TM, int WF, int EPI, bool SWH, int GS>
hipError_t run_skinny(const GemmArgs& a, bool vec, hipStream_t s) {
  // per-group: the workgroup's 16 columns of every group's scales in LDS
  const size_t lds = (EPI == EPI_PG) ? (size_t)(a.K / GS) * 16 * sizeof(float) : 0;
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  constexpr int kMaxKW = TM == 1 ? 16 : 8;
  const int64_t blocks = (a.N + 15) / 16;
  const int nkb = (a.K + 63) / 64;
  int kw = 4;
  if constexpr (EPI == EPI_PG) {
    const int G = a.K / GS;
    while (kw < kMaxKW && blocks * kw < 16 * 256 && G >= 2 * 2 * kw) kw *= 2;
    if (TM == 4 && kw == 8 && blocks > 256) kw = 4;
    // int8 weights, one row block, >= 512 column blocks: 4 waves per
    // workgroup (measured: N=12288 K=4096 M=16 gs 64: 27.7 vs 20.3 us at 8;
    // N=10240 K=2560 M=8: 19.3 vs 13.5 us).  int4 weights measured level.
    if (WF == W_I8 && TM == 1 && blocks >= 512) kw = 4;
    if constexpr (kMaxKW >= 16)
      if (kw == 16) return run_skinny_pg_kw<TM, WF, SWH, GS, 16>(a, vec, lds, s);
    if constexpr (kMaxKW >= 8)
      if (kw == 8) return run_skinny_pg_kw<TM, WF, SWH, GS, 8>(a, vec, lds, s);
    return run_skinny_pg_kw<TM, WF, SWH, GS, 4>(a, vec, lds, s);
  } else {
    while (kw < kMaxKW && blocks * kw < 16 * 256 && nkb >= 2 * kw * 4) kw *= 2;
    if (TM == 4 && kw == 8 && blocks > 256) kw = 4;
    if constexpr (kMaxKW >= 16)
      if (kw == 16) return run_skinny_kw<TM, WF, EPI, SWH, GS, 16>(a, vec, lds, s);
    if constexpr (kMaxKW >= 8)
      if (kw == 8) return run_skinny_kw<TM, WF, EPI, SWH, GS, 8>(a, vec, lds, s);
    return run_skinny_kw<TM, WF, EPI, SWH, GS, 4>(a, vec, lds, s);
  }
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
