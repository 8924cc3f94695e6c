// Small-M int8 GEMM (M <= 16, int8 weights, per-channel or int32 epilogue)
// as a weight stream through LDS.
//
// Semantics are those of the other GEMM kernels, bit for bit:
//   EPI_I32 cider/kernels/w8a8_matmul.metal:301-453
//   EPI_PC  cider/kernels/w8a8_matmul.metal:63-81 (int8 weights, with bias)
//
// MI355X layout
//   * A workgroup of KW = 4 waves owns RB blocks of 16 weight rows (n0 ..
//     n0 + 16 RB - 1) and every activation row (M <= MB, MB = 8 or 16).  K
//     arrives in stages of 512 bytes per row: the stage's weight rows and
//     activation rows go global -> LDS by global_load_lds_dwordx4, each 1 KB
//     instruction covering 512 contiguous bytes of two rows, into a ring of
//     NS stages.  Whole row pieces per instruction are what the vector-memory
//     path moves fastest; an MFMA operand load straight from HBM touches 16
//     rows x 64 B per instruction instead.  Every wave issues the same number
//     of loads per stage, so a stage is waited for by one constant vmcnt.
//   * LDS slot of 16-byte chunk c of row r (rows of 512 B): r * 512 +
//     16 * (c ^ (r % 16)).  The DMA lane that writes a slot fetches the chunk
//     that belongs there, so the 16 rows one operand read touches at a k-slice
//     fall in 16 distinct 16-byte bank groups.
//   * The four waves split each stage's eight 64-wide k-steps, two each, and
//     accumulate v_mfma_i32_16x16x64_i8 tiles (weights as A, activations as
//     B) in registers.  After the last stage the partial tiles are summed
//     through LDS (int32: exact in any order) and wave rb runs the epilogue of
//     block rb.
#include "common.hpp"
#include "dma_common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

constexpr int kSdBK = 512;   // k bytes per row and stage
constexpr int kSdKW = 4;     // waves per workgroup

template <int RB, int MB, int NS>
struct SdCfg {
  static constexpr int ROWS = 16 * RB;
  static constexpr int CPR = kSdBK / 16;              // 16-byte chunks per row
  static constexpr int WS = ROWS * kSdBK, XS = MB * kSdBK;
  static constexpr int STAGE = WS + XS;
  static constexpr int NWI = WS / 1024, NXI = XS / 1024;  // DMA instructions per stage
  static constexpr int PI = NWI + NXI;
  static constexpr int PW = PI / kSdKW;                // per wave and stage
  static constexpr int RING = NS * STAGE;
  static constexpr int RED = kSdKW * RB * 64 * 16;     // partial tiles
  static constexpr int SMEM = RING > RED ? RING : RED;
  static_assert(NWI % kSdKW == 0 && NXI % kSdKW == 0, "whole DMA instructions per wave");
  static_assert(RB <= kSdKW, "one wave per block in the epilogue");
  static_assert(NS >= 2 && (NS - 2) * PW <= 63, "vmcnt range");
  static_assert(SMEM <= kLdsBytes, "LDS budget");
};

// Waits for the oldest outstanding stage of this wave when `rem` (0 ..
// NS - 2) later stages have been issued after it.
template <int PW, int NS>
__device__ __forceinline__ void wait_stage(int rem) {
  if constexpr (NS > 2) {
    if (rem >= NS - 2) {
      wait_vmcnt<PW * (NS - 2)>();
      return;
    }
    if constexpr (NS > 3) {
      if (rem == 2) {
        wait_vmcnt<PW * 2>();
        return;
      }
    }
    if (rem == 1) {
      wait_vmcnt<PW>();
      return;
    }
  }
  wait_vmcnt<0>();
}

}  // namespace

template <int RB, int MB, int NS, int EPI>
__global__ __launch_bounds__(kSdKW * 64) void skinny_dma_kernel(const GemmArgs p) {
  using C = SdCfg<RB, MB, NS>;
  constexpr int PW = C::PW, CPR = C::CPR;
  __shared__ __attribute__((aligned(1024))) int8_t smem[C::SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int n0 = blockIdx.x * C::ROWS;
  const int nst = K / kSdBK;
  const int8_t* wbase = reinterpret_cast<const int8_t*>(p.w) + (int64_t)n0 * K;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  // Per-lane source offsets of this wave's PW instructions of a stage
  // (stage-invariant; a stage advances the scalar bases by 512).  Instruction
  // i = wave + KW j of the stage: the first NWI carry weight rows, the rest
  // activation rows, so j < NWI / KW decides which at compile time.
  constexpr int JW = C::NWI / kSdKW;
  uint32_t off[PW];
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int i = wave + kSdKW * j;
    const bool w = j < JW;
    const int s = (w ? i : i - C::NWI) * 64 + lane;  // LDS slot (16 B) in the block
    const int r = s / CPR, c = (s % CPR) ^ (r & 15);
    const int row = w ? min(n0 + r, N - 1) - n0 : min(r, M - 1);
    off[j] = (uint32_t)row * (uint32_t)K + 16u * (uint32_t)c;
  }
  auto issue = [&](int st) {
    const uint32_t slot = lds0 + (uint32_t)((st % NS) * C::STAGE);
    const int8_t* wsrc = wbase + (int64_t)st * kSdBK;
    const int8_t* xsrc = p.x + (int64_t)st * kSdBK;
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      const int i = wave + kSdKW * j;
      if (j < JW)
        dma16s(wsrc, off[j], __builtin_amdgcn_readfirstlane(slot + i * 1024));
      else
        dma16s(xsrc, off[j], __builtin_amdgcn_readfirstlane(slot + C::WS + (i - C::NWI) * 1024));
    }
  };

  i32x4 acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = i32x4{0, 0, 0, 0};

#pragma unroll
  for (int st = 0; st < NS - 1; ++st) issue(st);  // host: nst >= NS - 1
  for (int st = 0; st < nst; ++st) {
    wait_stage<PW, NS>(min(NS - 2, nst - 1 - st));
    __syncthreads();  // every wave's loads of stage st have landed; slot st-1 is free
    if (st + NS - 1 < nst) issue(st + NS - 1);
    const int8_t* slot = smem + (st % NS) * C::STAGE;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = 2 * wave + j;  // k-step of the stage
      const int cs = 16 * ((4 * t + lq) ^ lr);
      // activation row lr (lanes past MB re-read row lr - MB: columns past M
      // are not stored)
      const int xr = lr & (MB - 1);
      const i32x4 b = *reinterpret_cast<const i32x4*>(slot + C::WS + xr * kSdBK +
                                                      16 * ((4 * t + lq) ^ xr));
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(slot + (16 * rb + lr) * kSdBK + cs);
        acc[rb] = mfma_i8(a, b, acc[rb]);
      }
    }
  }

  // ---- the four partial tiles, summed through LDS
  __syncthreads();  // the ring is reused
  i32x4* red = reinterpret_cast<i32x4*>(smem);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) red[(wave * RB + rb) * 64 + lane] = acc[rb];
  __syncthreads();
  if (wave >= RB) return;
  const int rb = wave;
  i32x4 v4 = red[rb * 64 + lane];
#pragma unroll
  for (int w = 1; w < kSdKW; ++w) v4 += red[(w * RB + rb) * 64 + lane];
  // lane holds C[n][m] for n = n0 + 16 rb + 4 lq + r (r < 4), m = lr
  const int ncol = n0 + 16 * rb + 4 * lq;
  const int m = lr;
  if (ncol >= N || m >= M) return;
  if constexpr (EPI == EPI_I32) {
    *reinterpret_cast<i32x4*>(reinterpret_cast<int32_t*>(p.y) + (int64_t)m * N + ncol) = v4;
  } else {
    const float sam = p.sa[m];
    const f32x4 swv = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.sw) + ncol);
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = (float)v4[r] * sam;
      v[r] = v[r] * swv[r];
      if (p.bias) v[r] = v[r] + h2f(p.bias[ncol + r]);
    }
    *reinterpret_cast<i32x2*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + ncol) =
        i32x2{(int)f2h2(v[0], v[1]), (int)f2h2(v[2], v[3])};
  }
}

namespace {

template <int RB, int MB, int NS, int EPI>
hipError_t run_sd(const GemmArgs& a, hipStream_t s) {
  const int rows = 16 * RB;
  skinny_dma_kernel<RB, MB, NS, EPI><<<(a.N + rows - 1) / rows, kSdKW * 64, 0, s>>>(a);
  return hipGetLastError();
}

// The fewest blocks of 16 rows per workgroup whose grid fills at most one
// workgroup per CU (every workgroup reads all activation rows, so fewer,
// taller workgroups read them fewer times); 4 past three blocks per CU.
template <int MB, int EPI>
hipError_t pick_rb_sd(const GemmArgs& a, hipStream_t s) {
  const int cus = num_cus();
  const int blocks = (a.N + 15) / 16;
  if (blocks <= cus) return run_sd<1, MB, 4, EPI>(a, s);
  if (blocks <= 2 * cus) return run_sd<2, MB, 4, EPI>(a, s);
  if (blocks <= 3 * cus) return run_sd<3, MB, 4, EPI>(a, s);
  return run_sd<4, MB, 4, EPI>(a, s);
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// Shapes the kernel takes: 1 <= M <= 16, int8 weights, K % 512 == 0 with at
// least 3 stages (K >= 1536), K * 64 < 2^32, N % 4 == 0, 16-byte aligned
// operands.
bool skinny_dma_supported(const GemmArgs& a, int wf, int epi) {
  if (wf != W_I8 || epi == EPI_PG) return false;
  if (a.M < 1 || a.M > 16 || a.K % kSdBK != 0 || a.K / kSdBK < 3 || a.N % 4 != 0) return false;
  if ((int64_t)a.K * 64 >= ((int64_t)1 << 32)) return false;
  if (!al16(a.x) || !al16(a.w) || !al16(a.y)) return false;
  if (epi == EPI_PC && !al16(a.sw)) return false;
  return true;
}

hipError_t launch_skinny_dma(const GemmArgs& a, int epi, hipStream_t s) {
  if (epi == EPI_I32) {
    if (a.M <= 8) return pick_rb_sd<8, EPI_I32>(a, s);
    return pick_rb_sd<16, EPI_I32>(a, s);
  }
  if (a.M <= 8) return pick_rb_sd<8, EPI_PC>(a, s);
  return pick_rb_sd<16, EPI_PC>(a, s);
}

}  // namespace cider
