// Small-M int8 GEMM (2 <= M <= 64, and W4A8 at M == 1) as a weight stream:
// the regime where reading the weights from HBM sets the time.
//
// Semantics are those of the other GEMM kernels, bit for bit:
//   EPI_I32 cider/kernels/w8a8_matmul.metal:301-453
//   EPI_PC  cider/kernels/w8a8_matmul.metal:63-81 (int8 weights, with bias);
//           cider/kernels/w4a8_matmul.metal:47-89 (int4 weights, no bias)
//   EPI_PG  cider/kernels/pergroup_int8_gemm.metal:152-189: one sequential
//           fp32 chain per output over the groups in order
//
// MI355X layout
//   * A workgroup owns RB blocks of 16 weight rows (n0 .. n0 + 16 RB - 1) and
//     every activation row (TM blocks of 16); RB = 2 or 3 at M <= 16 on wide
//     N, so the activations of a k-range are read once for several blocks.  v_mfma_i32_16x16x64_i8 takes the weights as A (lane
//     l: row l % 16, k slice 16 (l / 16) of a 64-wide k-step) and the
//     quantized activations as B, so a lane's weight bytes go from HBM
//     straight into the MFMA operand.
//   * The workgroup's KW waves split the k-steps: contiguous ranges
//     (per-channel, int32), or whole groups dealt round-robin (per-group).  A
//     wave requests all of its k-steps' weights and activations at entry (at
//     most NB per lane), with clamped addresses so no load sits under a
//     branch (even under a wave-uniform branch the compiler waits for every
//     load issued before it); surplus slots re-read the wave's last k-step
//     and are not used.
//   * Per-channel / int32: each wave's int32 partial tile is summed with the
//     others through LDS (exact in any order) and wave 0 runs the epilogue.
//   * Per-group: each wave writes its groups' terms f32(f32(D_g) * sw[g, n])
//     to LDS, and after one barrier the owner of each output adds all G terms
//     in group order -- the reference's chain.  Groups are taken in phases of
//     at most 64 KB of terms (128 KB when RB > 1), each phase loading its own
//     k-steps.
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

template <bool SWH>
__device__ __forceinline__ f32x4 load_scale4(const void* base, int64_t idx) {
  if constexpr (SWH) {
    const i32x2 v = *reinterpret_cast<const i32x2*>(reinterpret_cast<const uint16_t*>(base) + idx);
    return f32x4{h2f((uint16_t)((uint32_t)v[0] & 0xffffu)), h2f((uint16_t)((uint32_t)v[0] >> 16)),
                 h2f((uint16_t)((uint32_t)v[1] & 0xffffu)), h2f((uint16_t)((uint32_t)v[1] >> 16))};
  } else {
    return *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + idx);
  }
}

constexpr int kTermBytes = 64 * 1024;  // LDS for one phase of per-group terms (RB == 1)

// int4 weights load pairs of k-steps (16 bytes per lane) unless a group
// boundary falls inside a pair (gs 64)
constexpr bool pair_slots(int WF, int EPI, int GS) {
  return WF == W_I4 && (EPI != EPI_PG || GS >= 128);
}

// LDS for the per-group terms of a phase: RB > 1 runs one workgroup per CU
// and takes 128 KB, so the groups of the shapes it serves fit one phase.
constexpr int term_bytes(int RB) { return RB == 1 ? kTermBytes : 2 * kTermBytes; }

// Groups per phase of the per-group kernel: the phase's terms fit
// term_bytes, and a wave's share (every KW-th group) fits its NB load slots.
constexpr int phase_groups(int TM, int WF, int EPI, int GS, int KW, int NB, int RB = 1) {
  const int slots = EPI == EPI_PG ? GS / (pair_slots(WF, EPI, GS) ? 128 : 64) : 1;
  const int by_lds = term_bytes(RB) / (RB * TM * 256 * 4);
  const int by_regs = KW * (NB / slots);
  return by_lds < by_regs ? by_lds : by_regs;
}

}  // namespace

template <int TM, int WF, int EPI, bool SWH, int GS, int KW, int NB, int RB>
__global__ __launch_bounds__(KW * 64) void skinny_stream_kernel(const GemmArgs p) {
  constexpr int kThreads = KW * 64;
  constexpr bool PG = EPI == EPI_PG;
  constexpr int SUB = PG ? GS / 64 : 1;     // k-steps per group
  constexpr int NOUT = RB * TM * 256;       // outputs of the workgroup (16 RB n x 16 TM m)
  // per-group: groups per phase -- the terms of a phase fit term_bytes and
  // each wave's share of them fits its NB load slots
  constexpr int GP = phase_groups(TM, WF, EPI, GS, KW, NB, RB);
  constexpr int RED = PG ? GP * NOUT * 4 : KW * NOUT * 4;
  __shared__ __attribute__((aligned(16))) uint8_t lds[RED];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 15, lq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int n0 = blockIdx.x * 16 * RB;
  const int8_t* __restrict__ X = p.x;
  const int8_t* __restrict__ W = reinterpret_cast<const int8_t*>(p.w);
  const int64_t ldw = (WF == W_I4) ? (K >> 1) : K;
  // load slots of KSTEP k (below): K / 64 or K / 128; block rb's weight row
  // of this lane (clamped)
  const int8_t* wrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) wrow[rb] = W + (int64_t)min(n0 + 16 * rb + lrow, N - 1) * ldw;
  const int8_t* xrow[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) xrow[b] = X + (int64_t)min(b * 16 + lrow, M - 1) * K;

  // Weight and activation fragments of k-step k.  int8: lane (r, q) holds
  // k in [64 k + 16 q, +16) of row r.  int4 with P2 (K % 128 == 0 and no
  // group boundary inside a 128-wide pair): a lane loads 16 bytes of one
  // row, the 32 nibbles of k in [128 p + 32 q, +32), and the pair's two
  // MFMAs take their first and second 16 (the activations are loaded at the
  // same k): loads of 8 bytes per lane (16 rows x 32 bytes per instruction)
  // measured 40 % slower per byte than 16 bytes.  Without P2, int4 lanes load
  // the 8 bytes of k in [64 k + 16 q, +16).
  constexpr bool P2 = pair_slots(WF, EPI, GS);
  constexpr int KSTEP = P2 ? 128 : 64;       // k per load slot
  constexpr int NX = P2 ? 2 : 1;             // MFMA k-steps per load slot
  auto load_k = [&](int k, i32x4 (&wv)[RB], i32x4 (&xv)[NX][TM]) {
    if constexpr (P2) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) wv[rb] = ld16_nt(wrow[rb] + k * 64 + 16 * lq);
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        xv[0][b] = ld16(xrow[b] + k * 128 + 32 * lq);
        xv[1][b] = ld16(xrow[b] + k * 128 + 32 * lq + 16);
      }
    } else {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if constexpr (WF == W_I4) {
          const i32x2 v = ld8_nt(wrow[rb] + k * 32 + 8 * lq);
          wv[rb] = i32x4{v[0], v[1], 0, 0};
        } else {
          wv[rb] = ld16_nt(wrow[rb] + k * 64 + 16 * lq);
        }
      }
#pragma unroll
      for (int b = 0; b < TM; ++b) xv[0][b] = ld16(xrow[b] + k * 64 + 16 * lq);
    }
  };
  // MFMA operand h (of NX) of a load slot
  auto operand = [&](const i32x4& wv, int h) -> i32x4 {
    if constexpr (WF == W_I4) {
      uint32_t o0, o1, o2, o3;
      unpack_w4_word((uint32_t)wv[2 * h], o0, o1);
      unpack_w4_word((uint32_t)wv[2 * h + 1], o2, o3);
      return i32x4{(int)o0, (int)o1, (int)o2, (int)o3};
    } else {
      return wv;
    }
  };

  if constexpr (!PG) {
    // ---- contiguous range of load slots of this wave, in rounds of NB
    // whose loads are all issued before the round's MFMAs
    const int nk = K / KSTEP;
    const int per = (nk + KW - 1) / KW;
    const int k0 = min(wave * per, nk), kend = min(k0 + per, nk);
    i32x4 acc[RB][TM];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int b = 0; b < TM; ++b) acc[rb][b] = i32x4{0, 0, 0, 0};
    for (int kr = k0; kr < kend; kr += NB) {
      const int cnt = min(NB, kend - kr);
      i32x4 wv[NB][RB], xv[NB][NX][TM];
      // unconditional: even a wave-uniform branch around a load makes the
      // compiler wait for the loads before it; surplus slots re-read the
      // round's last slot
#pragma unroll
      for (int j = 0; j < NB; ++j) load_k(kr + min(j, cnt - 1), wv[j], xv[j]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        // uniform (cnt is per wave; MFMAs ignore EXEC).  An if, not a break:
        // the loop must unroll, or the fragment arrays go to scratch memory
        if (j < cnt) {
#pragma unroll
          for (int h = 0; h < NX; ++h)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
              const i32x4 a = operand(wv[j][rb], h);
#pragma unroll
              for (int b = 0; b < TM; ++b) acc[rb][b] = mfma_i8(a, xv[j][h][b], acc[rb][b]);
            }
        }
      }
    }
    // ---- the KW partial tiles, summed through LDS (int32: exact)
    i32x4* red = reinterpret_cast<i32x4*>(lds);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int b = 0; b < TM; ++b) red[((wave * RB + rb) * TM + b) * 64 + lane] = acc[rb][b];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int b = 0; b < TM; ++b)
#pragma unroll
        for (int w = 1; w < KW; ++w) acc[rb][b] += red[((w * RB + rb) * TM + b) * 64 + lane];
    // lane holds C[n][m] for n = n0 + 16 rb + 4 lq + r (r < 4), m = 16 b + lrow
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int ncol = n0 + 16 * rb + 4 * lq;
      if (ncol >= N) continue;
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int m = b * 16 + lrow;
        if (m >= M) continue;
        if constexpr (EPI == EPI_I32) {
          *reinterpret_cast<i32x4*>(reinterpret_cast<int32_t*>(p.y) + (int64_t)m * N + ncol) =
              acc[rb][b];
        } else {
          const float sam = p.sa[m];
          const f32x4 swv = load_scale4<false>(p.sw, ncol);
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            v[r] = (float)acc[rb][b][r] * sam;
            v[r] = v[r] * swv[r];
            if (p.bias) v[r] = v[r] + h2f(p.bias[ncol + r]);
          }
          *reinterpret_cast<i32x2*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + ncol) =
              i32x2{(int)f2h2(v[0], v[1]), (int)f2h2(v[2], v[3])};
        }
      }
    }
  } else {
    // ---- per-group: phases of GP groups; wave w takes groups w, w + KW, ...
    // of the phase, SUB k-steps each; terms go to LDS [group][output]
    const int G = K / GS;
    float* terms = reinterpret_cast<float*>(lds);
    constexpr int OWN = (NOUT + kThreads - 1) / kThreads;
    float facc[OWN];
#pragma unroll
    for (int o = 0; o < OWN; ++o) facc[o] = 0.0f;
    constexpr int SLOTS = SUB * 64 / KSTEP;  // load slots per group
    constexpr int NG = NB / SLOTS;           // groups of one wave per phase (host: <= NG)
    for (int g0 = 0; g0 < G; g0 += GP) {
      const int gp = min(GP, G - g0);
      const int ng = (gp - wave + KW - 1) / KW;  // groups of this wave (>= 0)
      i32x4 wv[NB][RB], xv[NB][NX][TM];
      f32x4 sv[NG][RB];
#pragma unroll
      for (int q = 0; q < NG; ++q) {
        // unconditional (see above): surplus slots re-read a valid group
        const int gc = min(g0 + wave + KW * min(q, max(ng - 1, 0)), G - 1);
#pragma unroll
        for (int s = 0; s < SLOTS; ++s)
          load_k(gc * SLOTS + s, wv[q * SLOTS + s], xv[q * SLOTS + s]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          sv[q][rb] = load_scale4<SWH>(p.sw, (int64_t)gc * N + min(n0 + 16 * rb + 4 * lq, N - 4));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < NG; ++q) {
        if (q >= ng) continue;  // uniform; not a break (see above)
        i32x4 d[RB][TM];
#pragma unroll
        for (int s = 0; s < SLOTS; ++s)
#pragma unroll
          for (int h = 0; h < NX; ++h)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
              const i32x4 a = operand(wv[q * SLOTS + s][rb], h);
#pragma unroll
              for (int b = 0; b < TM; ++b)
                d[rb][b] = mfma_i8(a, xv[q * SLOTS + s][h][b],
                                   s + h == 0 ? i32x4{0, 0, 0, 0} : d[rb][b]);
            }
        const int gl = wave + KW * q;  // group within the phase
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int b = 0; b < TM; ++b) {
            f32x4 t;
#pragma unroll
            for (int e = 0; e < 4; ++e) t[e] = (float)d[rb][b][e] * sv[q][rb][e];
            *reinterpret_cast<f32x4*>(terms + ((gl * RB + rb) * TM + b) * 256 + lane * 4) = t;
          }
      }
      __syncthreads();
      // the chain: output idx adds the phase's terms in group order
#pragma unroll
      for (int o = 0; o < OWN; ++o) {
        const int idx = tid + o * kThreads;
        if (idx < NOUT)
          for (int g = 0; g < gp; ++g) facc[o] = facc[o] + terms[g * NOUT + idx];
      }
      __syncthreads();  // terms are rewritten by the next phase
    }
    // output idx = (rb, b, lane, e): weight row n0 + 16 rb + 4 (lane / 16) + e,
    // activation row 16 b + lane % 16 (the MFMA's C layout)
#pragma unroll
    for (int o = 0; o < OWN; ++o) {
      const int idx = tid + o * kThreads;
      if (idx >= NOUT) continue;
      const int rb = idx / (TM * 256), b = (idx >> 8) % TM, l = (idx >> 2) & 63, e = idx & 3;
      const int n = n0 + 16 * rb + 4 * (l >> 4) + e, m = b * 16 + (l & 15);
      if (m >= M || n >= N) continue;
      float v = facc[o] * p.sa[m];
      if (p.bias) v = v + h2f(p.bias[n]);
      reinterpret_cast<uint16_t*>(p.y)[(int64_t)m * N + n] = f2h(v);
    }
  }
}

namespace {

template <int TM, int WF, int EPI, bool SWH, int GS, int KW, int NB, int RB = 1>
hipError_t run_ss(const GemmArgs& a, hipStream_t s) {
  skinny_stream_kernel<TM, WF, EPI, SWH, GS, KW, NB, RB>
      <<<(a.N + 16 * RB - 1) / (16 * RB), KW * 64, 0, s>>>(a);
  return hipGetLastError();
}

// Row blocks per workgroup at M <= 16: every workgroup reads the activations
// of its k-range once for its RB blocks, so 3 blocks read a third of the
// activation bytes of 1 (for int4 weights at M = 16 those bytes are twice the
// weight bytes).  RB > 1 runs 8 waves of NB = 8 slots (4 pair slots) and
// keeps about 256 workgroups; per-group needs every group in one phase.
// Measured (kernel only, N=12288 K=4096 M=16, int4 gs 128): 9.9 us at RB = 3
// against 14.7 us at RB = 1.
template <int WF, int EPI, bool SWH, int GS>
int pick_rb(const GemmArgs& a) {
  constexpr int NB = pair_slots(WF, EPI, GS) ? 4 : 8;
  int rb = a.N >= 48 * 240 ? 3 : a.N >= 32 * 240 ? 2 : 1;
  if constexpr (EPI == EPI_PG) {
    const int G = a.K / GS;
    while (rb > 1 && (rb == 3 ? G > phase_groups(1, WF, EPI, GS, 8, NB, 3)
                              : G > phase_groups(1, WF, EPI, GS, 8, NB, 2)))
      --rb;
  }
  return rb;
}

// KW waves per workgroup, 4 or 8 (a 16-wave workgroup's 128 VGPRs per lane
// do not hold NB load slots of fragments): 4 while a wave's share fits one
// round of NB slots (per-group: every group in one phase), else 8.
template <int TM, int WF, int EPI, bool SWH, int GS>
hipError_t pick_kw(const GemmArgs& a, hipStream_t s) {
  constexpr bool P2 = pair_slots(WF, EPI, GS);
  constexpr int KSTEP = P2 ? 128 : 64;
  // load slots per lane and round: a pair slot holds twice the activations
  constexpr int NB0 = TM == 1 ? 16 : TM == 2 ? 12 : 8;
  constexpr int NB = P2 ? NB0 / 2 : NB0;
  if constexpr (TM == 1 && EPI != EPI_I32) {
    constexpr int NBR = P2 ? 4 : 8;
    const int rb = pick_rb<WF, EPI, SWH, GS>(a);
    if (rb == 3) return run_ss<TM, WF, EPI, SWH, GS, 8, NBR, 3>(a, s);
    if (rb == 2) return run_ss<TM, WF, EPI, SWH, GS, 8, NBR, 2>(a, s);
  }
  if constexpr (EPI == EPI_PG) {
    // 4 waves when every group fits one phase of theirs, else 8
    const int G = a.K / GS;
    if (G <= phase_groups(TM, WF, EPI, GS, 4, NB)) return run_ss<TM, WF, EPI, SWH, GS, 4, NB>(a, s);
    return run_ss<TM, WF, EPI, SWH, GS, 8, NB>(a, s);
  } else {
    const int nk = a.K / KSTEP;
    if ((nk + 3) / 4 <= NB) return run_ss<TM, WF, EPI, SWH, GS, 4, NB>(a, s);
    return run_ss<TM, WF, EPI, SWH, GS, 8, NB>(a, s);
  }
}

template <int TM>
hipError_t dispatch_ss(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s) {
  if (epi == EPI_I32) return pick_kw<TM, W_I8, EPI_I32, false, 0>(a, s);
  if (epi == EPI_PC) {
    if (wf == W_I4) return pick_kw<TM, W_I4, EPI_PC, false, 0>(a, s);
    return pick_kw<TM, W_I8, EPI_PC, false, 0>(a, s);
  }
  if (wf == W_I4) {
    if (gs == 64) return pick_kw<TM, W_I4, EPI_PG, true, 64>(a, s);
    return pick_kw<TM, W_I4, EPI_PG, true, 128>(a, s);
  }
  if (gs == 64) return pick_kw<TM, W_I8, EPI_PG, false, 64>(a, s);
  if (gs == 128) return pick_kw<TM, W_I8, EPI_PG, false, 128>(a, s);
  return pick_kw<TM, W_I8, EPI_PG, false, 256>(a, s);
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// Shapes the streaming small-M kernel takes: K % 64 == 0 (int4 per-channel
// or with groups of 128 or more: K % 128 == 0), K <= 16384, N % 4 == 0,
// 16-byte aligned x, w, y and scales.
bool skinny_stream_supported(const GemmArgs& a, int wf, int epi, int gs) {
  if (a.M < 1 || a.M > 64 || a.K % 64 != 0 || a.N % 4 != 0 || a.K > 16384) return false;
  if (wf == W_I4 && (epi != EPI_PG || gs >= 128) && a.K % 128 != 0) return false;
  if (!al16(a.x) || !al16(a.y) || !al16(a.w)) return false;
  if (epi != EPI_I32 && ((uintptr_t)a.sw & 15) != 0) return false;
  if (epi == EPI_PG && gs != 64 && gs != 128 && gs != 256) return false;
  if (epi == EPI_PG && wf == W_I4 && gs == 256) return false;
  return true;
}

hipError_t launch_skinny_stream(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s) {
  if (a.M <= 16) return dispatch_ss<1>(a, wf, epi, gs, s);
  if (a.M <= 32) return dispatch_ss<2>(a, wf, epi, gs, s);
  return dispatch_ss<4>(a, wf, epi, gs, s);
}

}  // namespace cider
