// Tiled int8 GEMM, main path for int8 weights with K % 128 == 0 and N % 8 == 0:
// operands stream global -> LDS by gfx950's 16-byte LDS-DMA loads through a
// 2-slot LDS ring of 128-byte k-stages, the MFMAs are v_mfma_i32_32x32x32_i8,
// and the fp16 tile is staged through LDS so the output is written in whole
// rows.
//
// Reference semantics are those of gemm.hip (same epilogues, same fp32
// operation order, bit-identical results):
//   EPI_I32 cider/kernels/w8a8_matmul.metal:301-453
//   EPI_PC  cider/kernels/w8a8_matmul.metal:63-81
// (Per-group stays on the register-staged kernel: its in-loop scale loads
// would make the compiler wait for every LDS-DMA load in flight.)
//
// MI355X design
//   * 256 threads = 4 waves (2 x 2); tile BM (m) x BN (n), BM, BN in
//     {64, 128, 256}, chosen per shape so the grid covers the 256 CUs; at
//     256 x 256 each wave owns a 128 x 128 sub-tile = 4 x 4 blocks of 32 x 32
//     (16 int32 accumulators per lane per block, 256 AGPRs).  Weights are the MFMA A operand,
//     activations the B operand.  128 x 128 per wave is the smallest wave
//     tile whose LDS fragment traffic (64 B/clk/CU at full MFMA rate) plus the
//     DMA fill (32 B/clk) stays inside LDS bandwidth (128 B/clk/CU).
//   * K advances 128 bytes per stage; stage s lives in LDS slot s % NS, with
//     NS = 2 at 256 x 256 up to 8 at 64 x 64 (as many stages as fit 128 KB).  Each
//     wave moves its share of a stage with global_load_lds_dwordx4 (one
//     instruction = 8 rows x 128 bytes, written contiguously to LDS at M0):
//     no VGPR staging, no ds_write.  The loads are issued from inline asm, so
//     the compiler does not wait for them; the kernel waits explicitly
//     (s_waitcnt vmcnt(per-stage loads x younger stages)) before the barrier
//     that publishes a stage.
//   * A stage is four 32-wide k sub-steps.  The fragments of the next
//     sub-step (8 ds_read_b128) are read while the current sub-step's 16
//     MFMAs run.  The one barrier per stage sits before sub-step 3 of stage
//     kt: it publishes stage kt + 1 (issued NS - 1 stages earlier) and frees
//     the slot of stage kt, which then receives stage kt + NS.  128-byte stages
//     halve the barriers and DMA issue slots per MFMA compared with 64-byte
//     stages (measured: 154 vs 161 us at M=4096, N=10240, K=2560).
//   * LDS rows are 128 bytes: chunk c of row r is stored in slot
//     c ^ (r & 7) ^ ((r >> 3) & 1), a function of r mod 16 that keeps the
//     16 rows of a fragment read in distinct banks; the DMA destination is
//     contiguous, so each lane picks the global chunk of the slot it writes.
//   * Epilogue (per-channel): each wave dequantizes its accumulators to fp16
//     into a BM x BN LDS tile (rows padded by 16 bytes), then the workgroup
//     stores whole 2*BN-byte rows with 16-byte lanes, so HBM sees full
//     128-byte lines instead of 32-byte row fragments.
//   * Rows past M or N are loaded from the last valid row (their results are
//     never stored); K % 128 == 0 is required, so there is no K tail.
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

__device__ __forceinline__ int swz16(int r) { return (r & 7) ^ ((r >> 3) & 1); }
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// 16 bytes per lane from global `src` to LDS at lds_base + 16 * lane.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(src), "s"(lds_base)
      : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most y * PS LDS-DMA loads of this wave are outstanding,
// y <= Y (the immediate must be a compile-time constant).
template <int PS, int Y>
__device__ __forceinline__ void wait_younger(int y) {
  if constexpr (Y == 0) {
    wait_vmcnt<0>();
  } else {
    if (y >= Y)
      wait_vmcnt<Y * PS>();
    else
      wait_younger<PS, Y - 1>(y);
  }
}

}  // namespace

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_dma_kernel(const GemmArgs p) {
  static_assert((BM == 64 || BM == 128 || BM == 256) && (BN == 64 || BN == 128 || BN == 256),
                "tile shape");
  constexpr int BK = 128;
  constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
  constexpr int W_BYTES = BN * BK, X_BYTES = BM * BK, STAGE = W_BYTES + X_BYTES;
  constexpr int WI = BN / 32, XI = BM / 32;  // DMA instructions (8 rows each) per wave
  constexpr int PS = WI + XI;                 // vmcnt units per stage
  // ring slots: as many 128-byte stages as fit in 128 KB (2..8), so small
  // tiles, whose stages carry little MFMA work, keep more loads in flight
  constexpr int NS0 = 131072 / STAGE;
  constexpr int NS = NS0 < 2 ? 2 : (NS0 > 8 ? 8 : NS0);
  constexpr int OUT_LD = BN * 2 + 16;
  constexpr int RING = NS * STAGE, OUT = BM * OUT_LD;
  __shared__ __attribute__((aligned(1024))) int8_t smem[RING > OUT ? RING : OUT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int M = p.M, N = p.N, K = p.K;

  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  constexpr int GROUP_M = 4;
  const int per_group = GROUP_M * tiles_n;
  const int grp = t / per_group;
  const int first_m = grp * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int m0 = (first_m + (t % per_group) % gm) * BM;
  const int n0 = ((t % per_group) / gm) * BN;

  // DMA: instruction i of this wave fills tile rows R0 = (wave*WI + i)*8 .. +8;
  // lane l writes row R0 + l/8, slot l%8 = chunk ^ swz(row mod 16).
  const int8_t* wsrc[WI];
  const int8_t* xsrc[XI];
  {
    const int rr = lane >> 3, slot = lane & 7;
    const int8_t* W = reinterpret_cast<const int8_t*>(p.w);
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int row = (wave * WI + i) * 8 + rr;
      const int chunk = slot ^ swz16(row & 15);
      const int n = min(n0 + row, N - 1);
      wsrc[i] = W + (int64_t)n * K + chunk * 16;
    }
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int row = (wave * XI + i) * 8 + rr;
      const int chunk = slot ^ swz16(row & 15);
      const int m = min(m0 + row, M - 1);
      xsrc[i] = p.x + (int64_t)m * K + chunk * 16;
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem);
  auto issue = [&](int kt) {
    const uint32_t sb = lds0 + (uint32_t)((kt % NS) * STAGE);
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < WI; ++i) dma16(wsrc[i] + k0, sb + (wave * WI + i) * 8 * BK);
#pragma unroll
    for (int i = 0; i < XI; ++i) dma16(xsrc[i] + k0, sb + W_BYTES + (wave * XI + i) * 8 * BK);
  };

  const int frow = lane & 31;
  const int fsw = swz16(lane & 15);
  auto read_sub = [&](int kt, int j, i32x4 (&wf)[TN], i32x4 (&xf)[TM]) {
    const int8_t* Ws = smem + (kt % NS) * STAGE;
    const int8_t* Xs = Ws + W_BYTES;
    const int fs = ((2 * j + (lane >> 5)) ^ fsw) << 4;
#pragma unroll
    for (int a = 0; a < TN; ++a)
      wf[a] = *reinterpret_cast<const i32x4*>(Ws + (wn * WN + a * 32 + frow) * BK + fs);
#pragma unroll
    for (int b = 0; b < TM; ++b)
      xf[b] = *reinterpret_cast<const i32x4*>(Xs + (wm * WM + b * 32 + frow) * BK + fs);
  };

  i32x16 acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;
  auto compute = [&](const i32x4 (&wf)[TN], const i32x4 (&xf)[TM]) {
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b) acc[a][b] = mfma32(wf[a], xf[b], acc[a][b]);
  };

  const int nk = K / BK;
  i32x4 wf0[TN], xf0[TM], wf1[TN], xf1[TM];
  if (nk > 0) {
    const int pre = min(nk, NS);
    for (int st = 0; st < pre; ++st) issue(st);
    wait_younger<PS, NS - 1>(pre - 1);
    __syncthreads();
    read_sub(0, 0, wf0, xf0);
  }
  // stage kt: sub-steps 0..3; the barrier before sub-step 3 publishes stage
  // kt+1 (issued NS-1 stages earlier) and frees the slot of stage kt, which
  // receives stage kt+NS.
  for (int kt = 0; kt < nk; ++kt) {
    read_sub(kt, 1, wf1, xf1);
    compute(wf0, xf0);
    read_sub(kt, 2, wf0, xf0);
    compute(wf1, xf1);
    read_sub(kt, 3, wf1, xf1);
    compute(wf0, xf0);
    if (kt + 1 < nk) {
      wait_younger<PS, NS - 2>(min(nk - 1, kt + NS - 1) - (kt + 1));
      __syncthreads();
      if (kt + NS < nk) issue(kt + NS);
      read_sub(kt + 1, 0, wf0, xf0);
    }
    compute(wf1, xf1);
  }

  // ---- epilogue: lane holds, per 32x32 block and group g, 4 consecutive n
  //      n = nblk + 8g + 4 (lane / 32) + [0..3] of row m = mblk + lane % 32
  const int h = lane >> 5;
  if constexpr (EPI == EPI_I32) {
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      const int m = m0 + wm * WM + b * 32 + frow;
      if (m >= M) continue;
#pragma unroll
      for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * WN + a * 32 + 8 * g + 4 * h;
          if (n < N)
            *reinterpret_cast<i32x4*>(reinterpret_cast<int32_t*>(p.y) + (int64_t)m * N + n) =
                i32x4{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2],
                      acc[a][b][4 * g + 3]};
        }
    }
  } else {
    __syncthreads();  // every wave is done with the ring: reuse it for the tile
    float sam[TM];
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      const int m = m0 + wm * WM + b * 32 + frow;
      sam[b] = m < M ? p.sa[m] : 0.0f;
    }
#pragma unroll
    for (int a = 0; a < TN; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nl = wn * WN + a * 32 + 8 * g + 4 * h;  // column in tile
        const int n = n0 + nl;
        float swv[4] = {0.f, 0.f, 0.f, 0.f}, bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (n < N) {  // N % 8 == 0 on this path: n < N implies n + 3 < N
          const f32x4 v = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.sw) + n);
#pragma unroll
          for (int r = 0; r < 4; ++r) swv[r] = v[r];
          if (p.bias) {
            const i32x2 bb = ld8(p.bias + n);
            bv[0] = h2f((uint16_t)((uint32_t)bb[0] & 0xffffu));
            bv[1] = h2f((uint16_t)((uint32_t)bb[0] >> 16));
            bv[2] = h2f((uint16_t)((uint32_t)bb[1] & 0xffffu));
            bv[3] = h2f((uint16_t)((uint32_t)bb[1] >> 16));
          }
        }
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const int ml = wm * WM + b * 32 + frow;  // row in tile
          uint16_t o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v = (float)acc[a][b][4 * g + r] * sam[b];
            v = v * swv[r];
            if (p.bias) v = v + bv[r];
            o[r] = f2h(v);
          }
          *reinterpret_cast<i32x2*>(smem + ml * OUT_LD + nl * 2) =
              i32x2{(int)(o[0] | ((uint32_t)o[1] << 16)), (int)(o[2] | ((uint32_t)o[3] << 16))};
        }
      }
    }
    __syncthreads();
    // whole rows: BN / 8 lanes x 16 bytes per row, 512 / BN rows per store
    constexpr int LPR = BN / 8, RPS = 64 / LPR;
    const int cl = (lane % LPR) * 8;  // first column of this lane's 8
    const int n = n0 + cl;
#pragma unroll 4
    for (int rr = wave * RPS + lane / LPR; rr < BM; rr += 4 * RPS) {
      const int m = m0 + rr;
      if (m < M && n < N)
        *reinterpret_cast<i32x4*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + n) =
            *reinterpret_cast<const i32x4*>(smem + rr * OUT_LD + cl * 2);
    }
  }
}

namespace {

template <int BM, int BN, int EPI>
hipError_t run_dma(const GemmArgs& a, hipStream_t s) {
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  gemm_dma_kernel<BM, BN, EPI><<<tiles, 256, 0, s>>>(a);
  return hipGetLastError();
}

template <int EPI>
hipError_t pick_tile(const GemmArgs& a, hipStream_t s) {
  // Estimated time = rounds of 256 workgroups x tile area / tile efficiency
  // (MFMA work per LDS byte falls with the tile); ties go to the larger tile.
  struct Cand { int bm, bn; double eff; };
  static const Cand cands[] = {{256, 256, 1.0}, {128, 256, 0.8}, {128, 128, 0.6},
                               {64, 128, 0.45}, {64, 64, 0.3}};
  int best = 0;
  double best_cost = 1e300;
  for (int i = 0; i < 5; ++i) {
    const int64_t tiles =
        (int64_t)((a.M + cands[i].bm - 1) / cands[i].bm) * ((a.N + cands[i].bn - 1) / cands[i].bn);
    const double cost = (double)((tiles + 255) / 256) * cands[i].bm * cands[i].bn / cands[i].eff;
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = i;
    }
  }
  switch (best) {
    case 0: return run_dma<256, 256, EPI>(a, s);
    case 1: return run_dma<128, 256, EPI>(a, s);
    case 2: return run_dma<128, 128, EPI>(a, s);
    case 3: return run_dma<64, 128, EPI>(a, s);
    default: return run_dma<64, 64, EPI>(a, s);
  }
}

}  // namespace

// Eligible: int8 weights, EPI_I32 or EPI_PC, K % 128 == 0, N % 8 == 0,
// 16-byte aligned operands.
hipError_t launch_gemm_dma(const GemmArgs& a, int epi, hipStream_t s) {
  if (epi == EPI_I32) return pick_tile<EPI_I32>(a, s);
  return pick_tile<EPI_PC>(a, s);
}

}  // namespace cider
