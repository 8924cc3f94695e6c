// Tiled int8 GEMM on CDNA4 MFMA with fused dequant epilogues.
//
//   y[m, n] = epilogue( sum_k x[m, k] * w[n, k] )      (int32 accumulation)
//
// Reference semantics (one kernel family here replaces three Metal ones):
//   EPI_I32 : raw int32 store          cider/kernels/w8a8_matmul.metal:301-453
//   EPI_PC  : h(((f32(acc)*sa[m])*sw[n]) [+ bias[n]])
//                                      cider/kernels/w8a8_matmul.metal:63-81
//                                      cider/kernels/w4a8_matmul.metal:83 (no bias)
//   EPI_PG  : acc_f = sum_g f32(f32(D_g)*sw[g,n]) sequentially in g, then
//             h((acc_f*sa[m]) [+ bias[n]])
//                                      cider/kernels/pergroup_int8_gemm.metal:152-189
//
// MI355X design
//   * 256 threads = 4 waves in a 2 (m) x 2 (n) grid; a workgroup owns a
//     BM x BN output tile, each wave a (BM/2) x (BN/2) sub-tile built from
//     v_mfma_i32_16x16x64_i8.  The weight tile is the MFMA "A" operand and the
//     activation tile the "B" operand, so a lane's four accumulators are four
//     consecutive output columns n of one row m: the epilogue stores 8 bytes
//     (4 x fp16) or 16 bytes (4 x int32) per lane.
//   * K advances 128 bytes per stage.  Global -> registers -> LDS with two
//     LDS buffers and one barrier per stage: the loads of stage k+1 are in
//     flight while stage k is multiplied.
//   * LDS tile rows are 128 bytes; 16-byte chunk c of row r sits at chunk
//     c ^ (r & 7) ^ ((r >> 3) & 1).  The swizzle depends on r mod 16 only (a
//     fragment row is 16-aligned base + lane % 16) and is injective on any 8
//     consecutive rows and on the 8 rows of either parity among 16, so the
//     row-wise ds_write_b128 stores and the column-wise ds_read_b128 fragment
//     loads are bank-conflict free for 32- and 64-bank LDS.
//   * Packed int4 weights are unpacked to int8 in registers between the
//     global load and the LDS store (once per weight byte per workgroup).
//   * Workgroups are remapped so each XCD works on a contiguous, grouped
//     range of tiles (L2 reuse of the x and w panels).
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

constexpr int kBK = 128;  // K bytes per stage
constexpr int kThreads = 256;

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kBK + ((chunk ^ swz(row)) << 4);
}

template <int BM, int BN>
struct TileCfg {
  static constexpr int WM = BM / 2, WN = BN / 2;  // per-wave sub-tile
  static constexpr int TM = WM / 16, TN = WN / 16;
  static constexpr int W_BYTES = BN * kBK;
  static constexpr int X_BYTES = BM * kBK;
  static constexpr int STAGE = W_BYTES + X_BYTES;
  static constexpr int XL = BM * 8 / kThreads;   // 16-byte x chunks per thread
  static constexpr int WL8 = BN * 8 / kThreads;  // 16-byte int8 w chunks
  static constexpr int WL4 = BN * 4 / kThreads;  // 16-byte packed int4 chunks
  static_assert(BM % 32 == 0 && BN % 64 == 0, "tile shape");
};

// Loads `nbytes` (<= 16) bytes at p; whole 16-byte vector when VEC.
template <bool VEC>
__device__ __forceinline__ i32x4 load_chunk(const int8_t* p, int nbytes) {
  if (nbytes <= 0) return i32x4{0, 0, 0, 0};
  if constexpr (VEC) {
    return ld16(p);
  } else {
    if (nbytes >= 16 && (((uintptr_t)p & 15) == 0)) return ld16(p);
    return load_bytes_partial(p, nbytes < 16 ? nbytes : 16);
  }
}

template <bool SWH>
__device__ __forceinline__ void load_scale4(const void* base, int64_t idx,
                                            int n, int N, bool vec, float out[4]) {
  if constexpr (SWH) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(base) + idx;
    if (vec) {
      const i32x2 v = ld8(p);
      out[0] = h2f((uint16_t)((uint32_t)v[0] & 0xffffu));
      out[1] = h2f((uint16_t)((uint32_t)v[0] >> 16));
      out[2] = h2f((uint16_t)((uint32_t)v[1] & 0xffffu));
      out[3] = h2f((uint16_t)((uint32_t)v[1] >> 16));
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = (n + r < N) ? h2f(p[r]) : 0.0f;
    }
  } else {
    const float* p = reinterpret_cast<const float*>(base) + idx;
    if (vec) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p);
      out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = (n + r < N) ? p[r] : 0.0f;
    }
  }
}

}  // namespace

// VEC: K % 16 == 0 (int8 w) or K % 32 == 0 (int4 w), N % 4 == 0 and every
// pointer 16-byte aligned; otherwise loads and stores are bounds-checked per
// byte / element.
template <int BM, int BN, int WF, int EPI, bool SWH, int GS, bool VEC>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(const GemmArgs p) {
  using C = TileCfg<BM, BN>;
  constexpr int TM = C::TM, TN = C::TN, WM = C::WM, WN = C::WN;
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar
  const int wm = wave & 1, wn = wave >> 1;
  const int M = p.M, N = p.N, K = p.K;

  // ---- tile index: XCD-contiguous, then grouped by GROUP_M rows of tiles
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  constexpr int GROUP_M = 4;
  const int per_group = GROUP_M * tiles_n;
  const int g = t / per_group;
  const int first_m = g * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int tb_m = first_m + (t % per_group) % gm;
  const int tb_n = (t % per_group) / gm;
  const int m0 = tb_m * BM, n0 = tb_n * BN;

  const int8_t* __restrict__ X = p.x;
  const int8_t* __restrict__ W = reinterpret_cast<const int8_t*>(p.w);
  const int64_t ldw = (WF == W_I4) ? (K >> 1) : K;  // bytes per weight row

  // ---- global -> register staging
  constexpr int WL = (WF == W_I4) ? C::WL4 : C::WL8;
  i32x4 xs[C::XL], ws[WL];
  auto gload = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < C::XL; ++i) {
      const int e = tid + kThreads * i, row = e >> 3, c = e & 7;
      const int m = m0 + row, kk = k0 + c * 16;
      const int nb = (m < M) ? K - kk : 0;
      xs[i] = load_chunk<VEC>(X + (int64_t)m * K + kk, nb);
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      if constexpr (WF == W_I4) {
        const int e = tid + kThreads * i, row = e >> 2, c4 = e & 3;
        const int n = n0 + row, kb = (k0 >> 1) + c4 * 16;
        const int nb = (n < N) ? (int)ldw - kb : 0;
        ws[i] = load_chunk<VEC>(W + (int64_t)n * ldw + kb, nb);
      } else {
        const int e = tid + kThreads * i, row = e >> 3, c = e & 7;
        const int n = n0 + row, kk = k0 + c * 16;
        const int nb = (n < N) ? K - kk : 0;
        ws[i] = load_chunk<VEC>(W + (int64_t)n * K + kk, nb);
      }
    }
  };
  auto lstore = [&](int buf) {
    int8_t* Ws = smem + buf * C::STAGE;
    int8_t* Xs = Ws + C::W_BYTES;
#pragma unroll
    for (int i = 0; i < C::XL; ++i) {
      const int e = tid + kThreads * i, row = e >> 3, c = e & 7;
      *reinterpret_cast<i32x4*>(Xs + lds_off(row, c)) = xs[i];
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      if constexpr (WF == W_I4) {
        const int e = tid + kThreads * i, row = e >> 2, c4 = e & 3;
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) unpack_w4_word((uint32_t)ws[i][j], o[2 * j], o[2 * j + 1]);
        *reinterpret_cast<i32x4*>(Ws + lds_off(row, 2 * c4)) =
            i32x4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
        *reinterpret_cast<i32x4*>(Ws + lds_off(row, 2 * c4 + 1)) =
            i32x4{(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
      } else {
        const int e = tid + kThreads * i, row = e >> 3, c = e & 7;
        *reinterpret_cast<i32x4*>(Ws + lds_off(row, c)) = ws[i];
      }
    }
  };

  i32x4 acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b) acc[a][b] = i32x4{0, 0, 0, 0};
  float facc[EPI == EPI_PG ? TN : 1][EPI == EPI_PG ? TM : 1][4];
  if constexpr (EPI == EPI_PG) {
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[a][b][r] = 0.0f;
  }

  const int lrow = lane & 15;
  const int lsw = swz(lrow);  // row & 15 == lrow for every fragment row
  const int nk = (K + kBK - 1) / kBK;
  const int ncol = n0 + wn * WN + 4 * (lane >> 4);  // first n of lane, tn = 0
  const bool vec_n = VEC;

  if (nk > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload(kt + 1);
    const int8_t* Ws = smem + (kt & 1) * C::STAGE;
    const int8_t* Xs = Ws + C::W_BYTES;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if constexpr (EPI == EPI_PG) {
        if (kt * kBK + s * 64 >= K) break;  // K % 64 == 0: last half stage
      }
      const int pos = ((s * 4 + (lane >> 4)) ^ lsw) << 4;
      i32x4 wf[TN], xf[TM];
#pragma unroll
      for (int a = 0; a < TN; ++a)
        wf[a] = *reinterpret_cast<const i32x4*>(Ws + (wn * WN + a * 16 + lrow) * kBK + pos);
#pragma unroll
      for (int b = 0; b < TM; ++b)
        xf[b] = *reinterpret_cast<const i32x4*>(Xs + (wm * WM + b * 16 + lrow) * kBK + pos);
      if constexpr (EPI == EPI_PG) {
        constexpr int SUB = GS / 64;  // 64-wide k steps per group
        const int ks = kt * 2 + s;    // global 64-wide k step
        const bool first = (ks % SUB) == 0;
        const bool last = (ks % SUB) == SUB - 1;
        float swv[TN][4];
        if (last) {
          const int64_t grow = (int64_t)(ks / SUB) * N;
#pragma unroll
          for (int a = 0; a < TN; ++a) {
            const int n = ncol + a * 16;
            if (n < N) {  // with vec_n, n < N implies n + 3 < N
              load_scale4<SWH>(p.sw, grow + n, n, N, vec_n, swv[a]);
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) swv[a][r] = 0.0f;
            }
          }
        }
        if (first) {  // uniform: a new group starts from a zero accumulator
#pragma unroll
          for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b) acc[a][b] = mfma_i8(wf[a], xf[b], i32x4{0, 0, 0, 0});
        } else {
#pragma unroll
          for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b) acc[a][b] = mfma_i8(wf[a], xf[b], acc[a][b]);
        }
        if (last) {
#pragma unroll
          for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float t = (float)acc[a][b][r] * swv[a][r];
                facc[a][b][r] = facc[a][b][r] + t;
              }
        }
      } else {
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
          for (int b = 0; b < TM; ++b) acc[a][b] = mfma_i8(wf[a], xf[b], acc[a][b]);
      }
    }
    if (kt + 1 < nk) lstore((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue
  float sam[TM];
  if constexpr (EPI != EPI_I32) {
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      const int m = m0 + wm * WM + b * 16 + lrow;
      sam[b] = m < M ? p.sa[m] : 0.0f;
    }
  }
#pragma unroll
  for (int a = 0; a < TN; ++a) {
    const int n = ncol + a * 16;
    if (n >= N) continue;
    float swv[4] = {0.f, 0.f, 0.f, 0.f}, bv[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (EPI == EPI_PC) load_scale4<false>(p.sw, n, n, N, vec_n, swv);
    if constexpr (EPI != EPI_I32) {
      if (p.bias) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bv[r] = (n + r < N) ? h2f(p.bias[n + r]) : 0.0f;
      }
    }
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      const int m = m0 + wm * WM + b * 16 + lrow;
      if (m >= M) continue;
      if constexpr (EPI == EPI_I32) {
        int32_t* yp = reinterpret_cast<int32_t*>(p.y) + (int64_t)m * N + n;
        if (vec_n) {
          *reinterpret_cast<i32x4*>(yp) = acc[a][b];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) yp[r] = acc[a][b][r];
        }
      } else {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (EPI == EPI_PC) {
            v[r] = (float)acc[a][b][r] * sam[b];
            v[r] = v[r] * swv[r];
          } else {
            v[r] = facc[a][b][r] * sam[b];
          }
          if (p.bias) v[r] = v[r] + bv[r];
        }
        const uint32_t o01 = f2h2(v[0], v[1]), o23 = f2h2(v[2], v[3]);
        uint16_t* yp = reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + n;
        if (vec_n) {
          *reinterpret_cast<i32x2*>(yp) = i32x2{(int)o01, (int)o23};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) yp[r] = (uint16_t)((r < 2 ? o01 : o23) >> (16 * (r & 1)));
        }
      }
    }
  }
}

// -------------------------------------------------------------------------
// host dispatch
// -------------------------------------------------------------------------

hipError_t launch_skinny(const GemmArgs& a, int wf, int epi, bool sw_half,
                         int gs, hipStream_t s);
hipError_t launch_gemm_dma(const GemmArgs& a, int epi, int wf, hipStream_t s);
hipError_t launch_gemm_dma_pg(const GemmArgs& a, int gs, bool sw_half, int wf, hipStream_t s);

namespace {

template <int BM, int BN, int WF, int EPI, bool SWH, int GS>
hipError_t run_tiled(const GemmArgs& a, bool vec, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (vec)
    gemm_kernel<BM, BN, WF, EPI, SWH, GS, true><<<tiles, kThreads, 0, s>>>(a);
  else
    gemm_kernel<BM, BN, WF, EPI, SWH, GS, false><<<tiles, kThreads, 0, s>>>(a);
  return hipGetLastError();
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

hipError_t launch_gemm(const GemmArgs& a, int wf, int epi, bool sw_half,
                       int gs, hipStream_t s) {
  // The GEMV on quantized activations for M <= 2.  At M = 3 and 4 the LDS
  // weight stream below was ahead on every shape measured (whole linears in
  // HIP graphs: per-channel N=10240 K=2560 M=4 9.9 against 13.5 us, per-group
  // gs 128 10.6 against 16.3 us, W4A8 N=12288 K=4096 10.4 against 14.5 us);
  // at M = 2 it was ahead on 7 of 10 shapes and up to 1.5 us behind on two.
  if (a.M <= 2 && gemv_q_supported(a, wf, false)) return launch_gemv_q(a, wf, epi, gs, s);
  const bool vec = (wf == W_I4 ? a.K % 32 == 0 : a.K % 16 == 0) && a.N % 4 == 0 &&
                   aligned16(a.x) && aligned16(a.w) && aligned16(a.y) &&
                   (a.sw == nullptr || aligned16(a.sw));
  // The LDS-DMA kernels address a tile's rows as a 64-bit base plus a 32-bit
  // per-lane offset of up to 256 rows * K bytes; longer rows take the
  // register-staged kernel, whose addresses are 64-bit throughout.
  const bool off32 = (int64_t)a.K * 256 < ((int64_t)1 << 32);
  const bool dma = epi != EPI_PG && (wf == W_I8 || epi == EPI_PC) && vec && a.K % 128 == 0 &&
                   a.N % 8 == 0 && off32;
  const bool dma_pg = epi == EPI_PG && (gs == 64 || gs == 128 || (gs == 256 && wf == W_I8)) &&
                      vec && a.K % 128 == 0 && a.K % gs == 0 && a.N % 8 == 0 && off32;
  if (a.M <= 64) {
    // The LDS-DMA kernel's 64 x 64 tiles load whole weight rows (one 16-byte
    // lane after another) and beat the skinny kernel, whose MFMA operand loads
    // touch 16 rows x 32-64 B, once they fill half the CUs or past M = 48
    // (N=12288 K=4096 M=16: 12.9 vs 18.7 us; N=4096 K=12288 M=16, 64 tiles:
    // 24.1 vs 17.1 us).
    // Per-group: the 128-row per-group DMA tiles (N / 64 of them at any M)
    // win once they fill half the CUs and M > 32, where the skinny kernel
    // moves to 4 row blocks per wave and 4 waves per workgroup (N=12288
    // K=4096 M=48, int8 gs 64: 45.1 vs 30.7 us; int4 gs 128: 36.2 vs 25.8 us),
    // and for int8 weights from the smallest M the shapes above do not take
    // (whole linears, int8 gs 64 N=10240 K=2560 M=17 / 24 / 32: 16.1 / 16.2
    // / 16.3 against 21.9 / 23.1 / 25.8 us on the skinny kernel; N=12288
    // K=4096: 22.6-23.0 against 26.3-29.4 us).  Below M = 32 the skinny kernel
    // keeps int4 weights (N=12288 K=4096 M=17, int4 gs 128: 22.8 against 29.0
    // us on the DMA tiles; gs 64 was split by shape).
    // M <= 16 with K % 512 == 0 (K >= 1536): the weight stream through LDS
    // (skinny_dma.hip), whole linears against the kernels below: int8
    // per-channel M=16 N=2560 K=10240 13.1 vs 19.0 us (64 x 64 DMA tiles);
    // int8 gs 64 N=10240 K=2560 11.2 vs 20.0 us, int4 gs 64 N=12288 K=4096
    // 14.2 vs 20.6 us and int4 gs 128 12.2 vs 12.5 us (register stream).
    // Other M <= 16 per-group or int4 shapes: the register weight stream
    // (skinny_stream.hip), ahead of the skinny and per-group DMA kernels
    // (N=12288 K=4096 M=16, int4 gs 128: 13.4 vs 17.2 us; int4 per-channel:
    // 11.5 vs 16.4 us; int8 gs 64: 18.3 vs 20.5 us).
    if (a.M <= 16 && skinny_dma_supported(a, wf, epi, sw_half, gs))
      return launch_skinny_dma(a, wf, epi, gs, s);
    if (a.M <= 16 && (epi == EPI_PG || wf == W_I4) && skinny_stream_supported(a, wf, epi, gs))
      return launch_skinny_stream(a, wf, epi, gs, s);
    if (dma && ((a.N + 63) / 64 >= 128 || a.M > 48)) return launch_gemm_dma(a, epi, wf, s);
    if (dma_pg && gs != 256 && (a.N + 63) / 64 >= 128 && (a.M > 32 || wf == W_I8))
      return launch_gemm_dma_pg(a, gs, sw_half, wf, s);
    return launch_skinny(a, wf, epi, sw_half, gs, s);
  }
  if (dma) return launch_gemm_dma(a, epi, wf, s);  // LDS-DMA pipeline (gemm_dma.hip)
  // per-group on the LDS-DMA per-group kernel (int4 weights at gs 256 --
  // which the W4A8 formats do not define -- and other shapes on the
  // register-staged kernel)
  if (dma_pg) return launch_gemm_dma_pg(a, gs, sw_half, wf, s);  // gemm_dma_pg.hip
  if (epi == EPI_I32) return run_tiled<256, 256, W_I8, EPI_I32, false, 0>(a, vec, s);
  if (epi == EPI_PC) {
    if (wf == W_I4) return run_tiled<256, 256, W_I4, EPI_PC, false, 0>(a, vec, s);
    return run_tiled<256, 256, W_I8, EPI_PC, false, 0>(a, vec, s);
  }
  // per-group
  if (wf == W_I4) {
    if (gs == 64) return run_tiled<256, 128, W_I4, EPI_PG, true, 64>(a, vec, s);
    return run_tiled<256, 128, W_I4, EPI_PG, true, 128>(a, vec, s);
  }
  if (gs == 64) return run_tiled<256, 128, W_I8, EPI_PG, false, 64>(a, vec, s);
  if (gs == 128) return run_tiled<256, 128, W_I8, EPI_PG, false, 128>(a, vec, s);
  return run_tiled<256, 128, W_I8, EPI_PG, false, 256>(a, vec, s);
}

}  // namespace cider
