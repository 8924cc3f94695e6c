// Tiled int8 GEMM, main path for int8 weights with K % 64 == 0 and N % 8 == 0:
// operands stream global -> LDS by gfx950's 16-byte LDS-DMA loads through a
// 4-slot LDS ring, the MFMAs are v_mfma_i32_32x32x32_i8, and the fp16 tile is
// staged through LDS so the output is written in whole rows.
//
// Reference semantics are those of gemm.hip (same epilogues, same fp32
// operation order, bit-identical results):
//   EPI_I32 cider/kernels/w8a8_matmul.metal:301-453
//   EPI_PC  cider/kernels/w8a8_matmul.metal:63-81
// (Per-group stays on the register-staged kernel: its in-loop scale loads
// would make the compiler wait for every LDS-DMA load in flight.)
//
// MI355X design
//   * 256 threads = 4 waves (2 x 2); tile 256 (m) x 256 (n); each wave owns
//     a 128 x 128 sub-tile = 4 x 4 blocks of 32 x 32 (16 int32 accumulators
//     per lane per block, 256 AGPRs).  Weights are the MFMA A operand,
//     activations the B operand.  128 x 128 per wave is the smallest wave
//     tile whose LDS fragment traffic (64 B/clk/CU at full MFMA rate) plus the
//     DMA fill (32 B/clk) stays inside LDS bandwidth (128 B/clk/CU).
//   * K advances 64 bytes per stage; stage s lives in LDS slot s % 4.  Each
//     wave moves its share of a stage with global_load_lds_dwordx4 (one
//     instruction = 16 rows x 64 bytes, written contiguously to LDS at M0):
//     no VGPR staging, no ds_write.  The loads are issued from inline asm, so
//     the compiler does not wait for them; the kernel waits explicitly with
//     s_waitcnt vmcnt(8 * younger stages) before the barrier that publishes a
//     stage.  Stage kt + 3 goes into the slot of stage kt - 1.
//   * A stage is two 32-wide k sub-steps.  The fragments of the next
//     sub-step (8 ds_read_b128) are read while the current sub-step's 16
//     MFMAs run; the barrier that publishes stage kt + 1 sits between the
//     two sub-steps of stage kt.
//   * LDS rows are 64 bytes: chunk c of row r is stored in slot
//     c ^ dswz(r mod 16), which keeps the 16 rows of a fragment read in
//     distinct banks; the DMA destination is contiguous, so each lane picks
//     the global chunk of the slot it writes.
//   * Epilogue (per-channel): each wave dequantizes its accumulators to fp16
//     into a 256 x 256 LDS tile (rows padded to 528 bytes), then the
//     workgroup stores whole 512-byte rows with 16-byte lanes, so HBM sees
//     full 128-byte lines instead of 32-byte row fragments.
//   * Rows past M or N are loaded from the last valid row (their results are
//     never stored); K % 64 == 0 is required, so there is no K tail.
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

constexpr int kDmaBK = 64;
constexpr int kDmaStages = 4;

__device__ __forceinline__ int dswz(int r) { return ((r >> 1) + (r >> 3)) & 3; }

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
  if constexpr (N == 0)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 4)
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else if constexpr (N == 6)
    asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if constexpr (N == 8)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (N == 12)
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else if constexpr (N == 16)
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if constexpr (N == 18)
    asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
  else if constexpr (N == 24)
    asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else
    static_assert(N < 0, "unsupported vmcnt");
}

}  // namespace


typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <int BN, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_dma_kernel(const GemmArgs p) {
  constexpr int BM = 256, BK = kDmaBK, NS = kDmaStages;
  constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
  constexpr int W_BYTES = BN * BK, X_BYTES = BM * BK, STAGE = W_BYTES + X_BYTES;
  constexpr int WI = BN / 64, XI = BM / 64;
  constexpr int PER_STAGE = WI + XI;
  constexpr int OUT_LD = BN * 2 + 16;  // bytes per staged output row
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

  const int8_t* wsrc[WI];
  const int8_t* xsrc[XI];
  {
    const int rr = lane >> 2, slot = lane & 3;
    const int chunk = slot ^ dswz(rr);
    const int8_t* W = reinterpret_cast<const int8_t*>(p.w);
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int n = min(n0 + (wave * WI + i) * 16 + rr, N - 1);
      wsrc[i] = W + (int64_t)n * K + chunk * 16;
    }
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int m = min(m0 + (wave * XI + i) * 16 + rr, M - 1);
      xsrc[i] = p.x + (int64_t)m * K + chunk * 16;
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem);
  auto issue = [&](int kt) {
    const uint32_t sb = lds0 + (uint32_t)((kt % NS) * STAGE);
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < WI; ++i) dma16(wsrc[i] + k0, sb + (wave * WI + i) * 16 * BK);
#pragma unroll
    for (int i = 0; i < XI; ++i) dma16(xsrc[i] + k0, sb + W_BYTES + (wave * XI + i) * 16 * BK);
  };

  // fragment of a 32-row block: lane reads row (lane % 32), 16-byte chunk
  // 2 * sub + lane / 32 of the 64-byte stage row
  const int frow = lane & 31;
  const int sw16 = dswz(lane & 15);
  const int fs0 = (((lane >> 5) + 0) ^ sw16) << 4;  // sub-step 0: chunks 0/1
  const int fs1 = (((lane >> 5) + 2) ^ sw16) << 4;  // sub-step 1: chunks 2/3
  auto read_sub = [&](int kt, int fs, i32x4 (&wf)[TN], i32x4 (&xf)[TM]) {
    const int8_t* Ws = smem + (kt % NS) * STAGE;
    const int8_t* Xs = Ws + W_BYTES;
#pragma unroll
    for (int a = 0; a < TN; ++a)
      wf[a] = *reinterpret_cast<const i32x4*>(Ws + (wn * WN + a * 32 + frow) * BK + fs);
#pragma unroll
    for (int b = 0; b < TM; ++b)
      xf[b] = *reinterpret_cast<const i32x4*>(Xs + (wm * WM + b * 32 + frow) * BK + fs);
  };
  auto wait_stage = [&](int need, int last_issued) {
    const int younger = last_issued - need;
    if (younger >= 3)
      wait_vmcnt<3 * PER_STAGE>();
    else if (younger == 2)
      wait_vmcnt<2 * PER_STAGE>();
    else if (younger == 1)
      wait_vmcnt<PER_STAGE>();
    else
      wait_vmcnt<0>();
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
    const int pre = min(nk, 3);
    for (int s = 0; s < pre; ++s) issue(s);
    wait_stage(0, pre - 1);
    __syncthreads();
    read_sub(0, fs0, wf0, xf0);
  }
  for (int kt = 0; kt < nk; ++kt) {
    // sub-step 0 of stage kt (F0) while reading sub-step 1 of stage kt (F1)
    read_sub(kt, fs1, wf1, xf1);
    compute(wf0, xf0);
    // publish stage kt + 1; its DMA was issued two stages ago
    if (kt + 1 < nk) {
      wait_stage(kt + 1, min(nk - 1, kt + 2));
      __syncthreads();
      if (kt + 3 < nk) issue(kt + 3);  // slot of stage kt - 1, fully read
      read_sub(kt + 1, fs0, wf0, xf0);
    }
    // sub-step 1 of stage kt (F1) while stage kt + 1 sub-step 0 loads (F0)
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
    // whole rows: 32 lanes x 16 bytes = one 512-byte row; two rows per store
    const int cl = (lane & 31) * 8;  // first column of this lane's 8
    const int n = n0 + cl;
#pragma unroll 4
    for (int rr = wave * 2 + (lane >> 5); rr < BM; rr += 8) {
      const int m = m0 + rr;
      if (m < M && n < N)
        *reinterpret_cast<i32x4*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + n) =
            *reinterpret_cast<const i32x4*>(smem + rr * OUT_LD + cl * 2);
    }
  }
}

namespace {

template <int BN, int EPI>
hipError_t run_dma(const GemmArgs& a, hipStream_t s) {
  const int tiles = ((a.M + 255) / 256) * ((a.N + BN - 1) / BN);
  gemm_dma_kernel<BN, EPI><<<tiles, 256, 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace

// Eligible: int8 weights, EPI_I32 or EPI_PC, K % 64 == 0, N % 8 == 0,
// 16-byte aligned operands.
hipError_t launch_gemm_dma(const GemmArgs& a, int epi, hipStream_t s) {
  if (epi == EPI_I32) return run_dma<256, EPI_I32>(a, s);
  return run_dma<256, EPI_PC>(a, s);
}

}  // namespace cider
