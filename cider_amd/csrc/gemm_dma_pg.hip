// Per-group int8 GEMM on the LDS-DMA pipeline (int8 or packed int4 weights,
// gs 64 / 128, and gs 256 for int8 weights; K % 128 == 0, N % 8 == 0).
//
// Reference semantics (cider/kernels/pergroup_int8_gemm.metal:90-191):
//   D_g[m,n] = sum over the gs k of group g of qa[m,k] * w[n,k]   (exact int32)
//   acc      = +0.0;  acc += float(D_g) * sw[g,n]  for g = 0, 1, ...
//   y[m,n]   = h(f32(acc * sa[m]) [+ f32(bias[n])])
// The reference compiles that flush under Metal's fast-math, which may
// contract it into a fused multiply-add, so its fp32 chain is defined up to
// the rounding of each product.  Here D_g is always exact, and the flush
// takes one of three forms:
//   * fma: acc = fma(f32(D_g), s, acc), 2 VALU ops per accumulator and group
//     (int8 weights with fp32 scales in both kernels; every format in the
//     one-set kernel), for tiles whose scales are all finite with |s| < 2^64
//     (pg_scales_tame, a workgroup vote after the prologue).  The result
//     differs from the two-rounding chain by the rounding of each product,
//     within the per-group bar of the tests.
//   * fast (fp16 scales in the two-set kernel): one fma per term from a
//     biased sum (below) rounds D_g * s once, bit-identical to the exact
//     chain, then the add: 2 VALU ops.
//   * exact: acc = acc + f32(f32(D_g) * s), the reference's operation order
//     with both roundings, 3 VALU ops: tiles with a non-finite or huge scale
//     (pg_exact_tile, straight from global memory; real weights' scales never
//     take it), and the two-set kernel where the fast flush's registers do
//     not fit.
// Split-K (mid M on small N): S K-slices of whole groups run the 64 x 64 tile
// into fp32 partial chains, and pg_splitk_sum_kernel adds the slices in slice
// order before the epilogue's fp32 operations.
//
// MI355X design
//   * Waves of 64 x 32 (TM = 2 blocks of 32 x 32 along m, TN = 1 along n),
//     v_mfma_i32_32x32x32_i8; operands reach LDS by global_load_lds_dwordx4
//     through a ring of 128-byte k-stages, with the constant-count waits,
//     swizzle and fixed-order sub-steps of the per-channel kernel
//     (gemm_dma.hip).  Three launch shapes: 128 x 128 tiles of 8 waves (two
//     per SIMD, 4 ring slots; gs 64 and 256 at M > 64), 128 x 64 tiles of
//     4 waves (gs 128 at two workgroups per CU, gs 64 at M <= 64), and 64 x 64
//     tiles of four 32 x 32 waves where those would leave most CUs idle (and
//     for the split-K slices).  gemm_dma_pg16_kernel below (one group set,
//     waves of 64 x 64) takes the grids of 512 tiles and more.
//   * Group accumulators: two int32 sets alternate by group.  A group's first
//     MFMA takes C = 0 (an inline constant), so starting a group costs
//     nothing.  While group g accumulates, group g-1 is flushed into the fp32
//     accumulators, a slice per sub-step interleaved with group g's MFMAs in
//     the same fixed order.  The flush bounds the kernel: at 2 VALU ops per
//     accumulator, 8 VALU ops per MFMA at gs = 128 and 16 at gs = 64, against
//     the MFMA's 32 cycles and 4 per wave64 VALU op.  A gs 256 group spans two
//     k-stages, so the sets alternate over a period of 4 stages instead of 2.
//     Before the first group the other set is zero and its "scales" are a
//     zero row, so the first flush adds +0.0; the last stage flushes the last
//     group after its MFMAs.  Every register is architectural (no AGPR reads
//     in the flush) and nothing spills: a spill reload is a vector-memory load
//     the compiler tracks, and waiting for it would also wait for every
//     LDS-DMA load in flight.
//   * Scales: wave 0 DMAs the scale rows of a stage's groups (sw[g, n0..n0+BN))
//     into an 8-slot LDS ring of its own, so a row stays in LDS until its
//     group has been flushed during the next stage.  Wave 0 therefore moves one
//     more load per stage than the others, and waits with its own count.
//   * Epilogue: sa and bias are requested during the last stage; acc * sa
//     (+ bias) is converted to fp16, staged in LDS and stored in whole rows
//     (a split-K slice stores its fp32 chains instead).
#include "common.hpp"
#include "dma_common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace cider {

namespace {

// Geometry of a BM x BN tile, WGM x WGN waves of (BM / WGM) x (BN / WGN);
// int8 or packed int4 weights (WF); OCC workgroups per CU share the LDS.
template <int BM, int BN_, int WF, int OCC, int WGM, int WGN>
struct PgCfg {
  static constexpr int BN = BN_, BK = 128, NW = WGM * WGN;
  static constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
  static constexpr int CH = BK / 16, RPI = 1024 / BK;        // X: 8 chunks, 8 rows per DMA
  static constexpr int WB = (WF == W_I4) ? BK / 2 : BK;      // weight bytes per row and stage
  static constexpr int CHW = WB / 16, RPIW = 1024 / WB;
  static constexpr int WI = BN / RPIW / NW;                  // DMA instructions (W rows)
  static constexpr int XI = BM / RPI / NW;                   // DMA instructions (X rows)
  static constexpr int PS = WI + XI;                         // per wave and stage (+1 on wave 0)
  static constexpr int W_BYTES = BN * WB;
  static constexpr int STAGE = W_BYTES + BM * BK;
  static constexpr int SSLOT = 1024, SNS = 8;                // scale ring
  static constexpr int LDS = kLdsBytes / OCC;
  static constexpr int NS0 = (LDS - SNS * SSLOT) / STAGE;
  static constexpr int NS = NS0 > 4 ? 4 : NS0;               // operand ring
  static constexpr int RING = NS * STAGE;
  static constexpr int SMEM = RING + SNS * SSLOT;
  static constexpr int OUT_LD = BN * 2 + 16;
  static constexpr int OUT = BM * OUT_LD;
  static_assert(WI >= 1 && XI >= 1 && TN >= 1 && TM >= 1, "tile too small for the DMA split");
  static_assert(WI * RPIW * NW == BN && XI * RPI * NW == BM, "whole DMA instructions");
  static_assert(64 * NW >= BM && 64 * NW >= BN, "one thread per tile row / column in the epilogue");
  static_assert(OUT + BM * 4 + BN * 2 <= RING, "epilogue staging fits the ring");
  static_assert(SMEM <= LDS, "LDS budget");
  static_assert(NS >= 2 && (NS - 1) * (PS + 1) <= 63, "vmcnt range");
};

// 8 bytes of packed int4 (element 2i in the low nibble of byte i) -> 16 int8
// in element order.
__device__ __forceinline__ i32x4 pg_unpack_w4_8(uint32_t w0, uint32_t w1) {
  uint32_t a, b, c, d;
  unpack_w4_word(w0, a, b);
  unpack_w4_word(w1, c, d);
  return i32x4{(int)a, (int)b, (int)c, (int)d};
}

template <int V>
using ic = std::integral_constant<int, V>;

// Fast flush (fp16 group scales).  A group's int32 sum D starts from the bit
// pattern of B = 1.5 * 2^23 instead of 0, so for |D| <= 2^22 (every group
// size here: |D| <= 128 * 128 * 256 = 2^22) the sum's bits read as the float
// F = B + D exactly.  For an fp16 scale s (11 significant bits) c = -B * s is
// exact in fp32, so fma(F, s, c) = round(D * s): the same single rounding as
// f32(f32(D) * s), since f32(D) is exact.  The conversion disappears from
// the flush: 2 VALU ops per accumulator instead of 3.  A non-finite s gives
// NaN where the specified product is +-inf; the kernel then redoes the tile
// with the exact flush.
constexpr int32_t kPgBiasBits = 0x4B400000;
constexpr float kPgBias = 12582912.0f;  // 1.5 * 2^23
static_assert(__builtin_bit_cast(float, kPgBiasBits) == kPgBias, "bias bits");

// fp16 element i of 4 packed in two words, widened (the fma takes it as an
// fp16 operand).
__device__ __forceinline__ float pg_half(const uint32_t (&r)[2], int i) {
  return (float)__builtin_bit_cast(f16x2, r[i >> 1])[i & 1];
}

// Width of the 4-wave tile (128 x 64).  gs = 128 runs two of its workgroups
// per CU: each workgroup's waits hide behind the other's flush.
constexpr int PG_LAUNCH_BN = 64;

}  // namespace

// Whether every group scale of columns [n0, n0 + BN) (sw [G, N], fp32 or fp16)
// is finite with |s| < 2^64.  Then |D_g * s| < 2^22 * 2^64 and no term or
// running sum of the exact or the fma flush comes near the binary32 range
// (K < 2^24), so neither chain meets an infinity or NaN, and the fma flush
// differs from the exact one by the rounding of each product alone.  Each
// thread reads 16-byte chunks of the block (L2-resident: every tile of the
// column reads it); the caller votes over the workgroup.
template <int BN, bool SWH>
__device__ __forceinline__ bool pg_scales_tame(const GemmArgs& p, int n0, int G, int nthreads) {
  constexpr int ESZ = SWH ? 2 : 4, PER16 = 16 / ESZ, CPRS = BN / PER16;
  const int N = p.N, tid = threadIdx.x;
  const int total = G * CPRS;
  uint32_t mx = 0;
  for (int c0 = 0; c0 < total; c0 += 8 * nthreads) {
    i32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = min(c0 + u * nthreads + tid, total - 1);
      const int g = idx / CPRS, col = min(n0 + (idx % CPRS) * PER16, N - PER16);
      v[u] = *reinterpret_cast<const i32x4*>(reinterpret_cast<const int8_t*>(p.sw) +
                                             ((int64_t)g * N + col) * ESZ);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = (uint32_t)v[u][e];
        if constexpr (SWH)
          mx = max(mx, max(w & 0x7fffu, (w >> 16) & 0x7fffu));
        else
          mx = max(mx, w & 0x7fffffffu);
      }
  }
  return SWH ? mx < 0x7c00u : mx < 0x5f800000u;  // fp16 finite / fp32 below 2^64
}

// The exact per-group chain for one BM x BN tile, straight from global
// memory: each thread computes whole outputs (v_dot4 int32 group sums, then
// acc = acc + f32(f32(D_g) * s) in group order, y = h(f32(acc * sa) [+ bias])).
// The fallback of the fma-flush kernels for tiles whose scales are not all
// finite and below 2^64; real weights' scales never are, so its speed does
// not matter, only its results.  `kbeg`, `kend`: the k range (a split-K
// slice), `part`: fp32 partial sums [M, N] of that slice instead of y.
template <int BM, int BN, int GS, bool SWH, int WF>
__device__ __forceinline__ void pg_exact_tile(const GemmArgs& p, int m0, int n0,
                                                        int nthreads, int kbeg = 0,
                                                        int kend = -1, float* part = nullptr) {
  constexpr bool W4 = (WF == W_I4);
  const int M = p.M, N = p.N, K = p.K;
  if (kend < 0) kend = K;
  const int64_t ldw = W4 ? (K >> 1) : K;
  for (int idx = threadIdx.x; idx < BM * BN; idx += nthreads) {
    const int m = m0 + idx / BN, n = n0 + idx % BN;
    if (m >= M || n >= N) continue;
    const int8_t* xr = p.x + (int64_t)m * K;
    const int8_t* wr = reinterpret_cast<const int8_t*>(p.w) + (int64_t)n * ldw;
    float acc = 0.0f;
    for (int g = kbeg / GS; g < kend / GS; ++g) {
      int32_t d = 0;
      for (int k = g * GS; k < (g + 1) * GS; k += 8) {
        const i32x2 xv = ld8(xr + k);
        uint32_t w0, w1;
        if constexpr (W4) {
          unpack_w4_word(*reinterpret_cast<const uint32_t*>(wr + k / 2), w0, w1);
        } else {
          const i32x2 wv = ld8(wr + k);
          w0 = (uint32_t)wv[0];
          w1 = (uint32_t)wv[1];
        }
        d = __builtin_amdgcn_sdot4(xv[0], (int)w0, d, false);
        d = __builtin_amdgcn_sdot4(xv[1], (int)w1, d, false);
      }
      const int64_t si = (int64_t)g * N + n;
      const float sc = SWH ? h2f(reinterpret_cast<const uint16_t*>(p.sw)[si])
                           : reinterpret_cast<const float*>(p.sw)[si];
      const float t = (float)d * sc;
      acc = acc + t;
    }
    if (part) {
      part[(int64_t)m * N + n] = acc;
    } else {
      float v = acc * p.sa[m];
      if (p.bias) v = v + h2f(p.bias[n]);
      reinterpret_cast<uint16_t*>(p.y)[(int64_t)m * N + n] = f2h(v);
    }
  }
}

// ks > 0: split-K.  Workgroup (t, s) runs tile t over k in [s ks, (s+1) ks)
// (whole groups and k-stages) and writes its fp32 group chain, before the
// per-token scale, to part + s M N; pg_splitk_sum_kernel adds the slices.
template <int BM, int BN, int GS, bool SWH, int WF, int OCC, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void gemm_dma_pg_kernel(const GemmArgs pin,
                                                                          int ks, float* part) {
  static_assert(GS == 64 || GS == 128 || GS == 256, "group size");
  using C = PgCfg<BM, BN, WF, OCC, WGM, WGN>;
  constexpr int NW = C::NW;
  constexpr bool W4 = (WF == W_I4);
  constexpr int WB = C::WB, CHW = C::CHW, RPIW = C::RPIW;
  constexpr int PG_BM = BM, PG_BN = C::BN, PG_BK = C::BK, PG_WM = C::WM, PG_WN = C::WN;
  constexpr int PG_TM = C::TM, PG_TN = C::TN, PG_CH = C::CH, PG_RPI = C::RPI;
  constexpr int PG_WI = C::WI, PG_XI = C::XI, PG_PS = C::PS, PG_W_BYTES = C::W_BYTES;
  constexpr int PG_STAGE = C::STAGE, PG_NS = C::NS, PG_RING = C::RING, PG_SSLOT = C::SSLOT;
  constexpr int PG_SNS = C::SNS, PG_SMEM = C::SMEM, PG_OUT_LD = C::OUT_LD, PG_OUT = C::OUT;
  constexpr int SUBG = GS / 32;              // k sub-steps per group (a stage has 4)
  constexpr int SRPS = SUBG < 4 ? 4 / SUBG : 1;  // scale rows a stage brings: its groups
  // stages per period of the set alternation (group parities compile-time):
  // 2, or 4 when a group spans two stages (gs 256)
  constexpr int PER = SUBG < 8 ? 2 : 4;
  constexpr int ESZ = SWH ? 2 : 4;           // scale element bytes
  constexpr int CPR = PG_BN * ESZ / 16;      // 16-byte chunks per scale row
  constexpr int ROWB = PG_BN * ESZ;          // bytes per scale row in LDS
  constexpr int NMF = PG_TN * PG_TM;         // MFMAs per sub-step
  constexpr int NR = PG_TN + PG_TM;          // fragment reads per sub-step
  constexpr int NCOMBO = PG_TN * 4;          // (block a, quad q) scale combos
  constexpr int NE = PG_TN * PG_TM * 16;     // accumulators of a set, per lane
  constexpr int EPS = NE / SUBG;             // accumulators flushed per sub-step
  static_assert(EPS % NMF == 0, "flush split");
  static_assert(CPR * 16 * SRPS <= PG_SSLOT && 64 / CPR >= SRPS, "scale rows per stage");
  static_assert(NCOMBO % 4 == 0, "whole combos per sub-step");
  // The flush before the first group (zero sums) reads zero "scales": 0 * s
  // would be NaN for an infinite s.  They sit in the last scale slot, whose
  // first DMA (stage SNS-1) is issued in stage SNS-1-NS, after every read of
  // the zero row (stages 0 and 1) has finished; each pass writes them anew.
  constexpr int kZeroRow = PG_RING + (PG_SNS - 1) * PG_SSLOT;
  static_assert(PG_SNS - 1 - PG_NS >= 2 && ROWB <= PG_SSLOT, "zero row slot");
  __shared__ __attribute__((aligned(1024))) int8_t smem[PG_SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WGM, wn = wave / WGM;
  const int h = lane >> 5;
  // K is the row pitch; the k-loop covers KL of it (a split-K slice: the
  // operands and scales start at the slice, and the partial sums go to pp)
  GemmArgs p = pin;
  float* pp = nullptr;
  if (ks > 0) {
    const int sl = blockIdx.y;
    p.x = pin.x + (int64_t)sl * ks;
    p.w = reinterpret_cast<const int8_t*>(pin.w) + (int64_t)sl * (W4 ? ks / 2 : ks);
    p.sw = reinterpret_cast<const int8_t*>(pin.sw) + (int64_t)(sl * (ks / GS)) * pin.N * ESZ;
    pp = part + (int64_t)sl * pin.M * pin.N;
  }
  const int M = p.M, N = p.N, K = p.K;
  const int KL = ks > 0 ? ks : K;
  const int G = KL / GS;
  const int nk = KL / PG_BK;
  int m0, n0;
  tile_coords<PG_BM, PG_BN>(xcd_remap(blockIdx.x, gridDim.x), M, 0, N, m0, n0);

  // Sources: the tile's first W (X) row as a wave-uniform base, and per
  // lane and instruction a 32-bit byte offset from it (< 256 rows x K).
  const int64_t ldw = W4 ? (K >> 1) : K;
  const int8_t* const wbase = reinterpret_cast<const int8_t*>(p.w) + (int64_t)n0 * ldw;
  const int8_t* const xbase = p.x + (int64_t)m0 * K;
  uint32_t woff[PG_WI], xoff[PG_XI];
#pragma unroll
  for (int i = 0; i < PG_WI; ++i) {
    const int row = (wave * PG_WI + i) * RPIW + lane / CHW;
    woff[i] = (uint32_t)((int64_t)(min(n0 + row, N - 1) - n0) * ldw +
                         ((lane % CHW) ^ swz<WB>(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < PG_XI; ++i) {
    const int row = (wave * PG_XI + i) * PG_RPI + lane / PG_CH;
    xoff[i] = (uint32_t)((int64_t)(min(m0 + row, M - 1) - m0) * K +
                         ((lane % PG_CH) ^ swz<PG_BK>(row)) * 16);
  }
  // scale DMA (wave 0): lane l moves chunk l % CPR of row l / CPR of a stage's
  // scale block; rows past the stage's groups (or past G) repeat a valid row
  const int srow = lane / CPR;
  const int8_t* ssrc =
      reinterpret_cast<const int8_t*>(p.sw) +
      (int64_t)min(n0 + (lane % CPR) * (16 / ESZ), N - 16 / ESZ) * ESZ;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem);

  auto dma_stage = [&](int st, int slot) __attribute__((always_inline)) {
    const uint32_t sb = lds0 + (uint32_t)(slot * PG_STAGE);
#pragma unroll
    for (int i = 0; i < PG_WI; ++i)
      dma16s(wbase + (int64_t)st * WB, woff[i], sb + (wave * PG_WI + i) * 1024);
#pragma unroll
    for (int i = 0; i < PG_XI; ++i)
      dma16s(xbase + (int64_t)st * PG_BK, xoff[i], sb + PG_W_BYTES + (wave * PG_XI + i) * 1024);
  };
  auto dma_one = [&](int st, int slot, int d) __attribute__((always_inline)) {
    const uint32_t sb = lds0 + (uint32_t)(slot * PG_STAGE);
    if (d < PG_WI)
      dma16s(wbase + (int64_t)st * WB, woff[d < PG_WI ? d : 0], sb + (wave * PG_WI + d) * 1024);
    else
      dma16s(xbase + (int64_t)st * PG_BK, xoff[d >= PG_WI ? d - PG_WI : 0],
             sb + PG_W_BYTES + (wave * PG_XI + d - PG_WI) * 1024);
  };
  // scale row(s) of stage st: the SRPS groups starting in it (gs 256: the
  // group it belongs to, also on its second stage, whose slot is not read)
  auto dma_scales = [&](int st) __attribute__((always_inline)) {
    const int g = min(st * 4 / SUBG + srow, G - 1);
    dma16(ssrc + (int64_t)g * N * ESZ, lds0 + PG_RING + (uint32_t)((st % PG_SNS) * PG_SSLOT));
  };

  // k mapping of sub-step j for lane half h (the same for both operands):
  //   int8 weights: k in [32 j + 16 h, + 16)               (X chunk 2j + h)
  //   int4 weights: k in [64 (j/2) + 32 h + 16 (j%2), + 16) (X chunk
  //     4 (j/2) + 2h + j%2; the W4 chunk 2 (j/2) + h holds the pair's 32
  //     nibbles, read once per pair, half j%2 unpacked per sub-step)
  const int frow = lane & 31;
  auto read_x = [&](int slot, int j, int b, i32x4 (&xfn)[PG_TM]) __attribute__((always_inline)) {
    const int8_t* Xs = smem + slot * PG_STAGE + PG_W_BYTES;
    const int row = wm * PG_WM + b * 32 + frow;
    const int c = W4 ? 4 * (j / 2) + 2 * h + (j % 2) : 2 * j + h;
    xfn[b] = *reinterpret_cast<const i32x4*>(Xs + row * PG_BK + ((c ^ swz<PG_BK>(row)) << 4));
  };
  auto read_w = [&](int slot, int j, int a, i32x4 (&dst)[PG_TN]) __attribute__((always_inline)) {
    const int8_t* Ws = smem + slot * PG_STAGE;
    const int row = wn * PG_WN + a * 32 + frow;
    const int c = W4 ? 2 * (j / 2) + h : 2 * j + h;
    dst[a] = *reinterpret_cast<const i32x4*>(Ws + row * WB + ((c ^ swz<WB>(row)) << 4));
  };
  i32x4 raw[PG_TN];  // int4 only: packed chunks of the current sub-step pair
  auto unpack_half = [&](int a, int half, i32x4 (&dst)[PG_TN]) __attribute__((always_inline)) {
    dst[a] = half == 0 ? pg_unpack_w4_8((uint32_t)raw[a][0], (uint32_t)raw[a][1])
                       : pg_unpack_w4_8((uint32_t)raw[a][2], (uint32_t)raw[a][3]);
  };

  float facc[PG_TN][PG_TM][16];
  float sa_t = 0.0f;
  uint16_t b_t = 0;

  // One pass over K into facc: prologue, k-loop and the last group's flush.
  // MODE 0: the exact flush; 1 (FAST, fp16 scales only): the biased sums
  // (kPgBiasBits), also exact; 2 (FMA, fp32 scales): facc = fma(f32(D), s,
  // facc) for tiles whose scales pass pg_scales_tame (else the tile runs
  // pg_exact_tile and kpass returns false: y is written, no epilogue).
  auto kpass = [&](auto modec) __attribute__((always_inline)) -> bool {
    constexpr int MODE = decltype(modec)::value;
    constexpr bool FAST = MODE == 1, FMA = MODE == 2;
    // Two int32 group sets alternate by group (set = group parity); while
    // group g accumulates, group g-1 is flushed, EPS of its accumulators per
    // sub-step over the SUBG sub-steps of group g (accumulator e of a set:
    // combo e / EPC, block (e / 4) % TM, element e % 4 of the combo's quad).
    // Before the first group the other set holds a zero sum and its "scales"
    // are the zero row, so that flush adds +0.0.
    constexpr int EPC = PG_TM * 4;          // accumulators per (a, q) combo
    constexpr int CPF = EPS >= EPC ? EPS / EPC : 1;  // combos of one sub-step's flush
    constexpr int EPM = EPS / NMF;          // accumulators flushed after each MFMA
    static_assert(EPS % EPC == 0 || EPC % EPS == 0, "flush split");
    static_assert(!FAST || SWH, "the fast flush needs fp16 scales");
    // A group's sum starts from C0: 0, or the fast flush's bias bit pattern.
    constexpr int32_t C0 = FAST ? kPgBiasBits : 0;
    i32x16 cinit;
#pragma unroll
    for (int r = 0; r < 16; ++r) cinit[r] = C0;
    i32x16 D[2][PG_TN][PG_TM];
#pragma unroll
    for (int a = 0; a < PG_TN; ++a)
#pragma unroll
      for (int b = 0; b < PG_TM; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          D[0][a][b][r] = C0;
          D[1][a][b][r] = C0;
          facc[a][b][r] = 0.0f;
        }

    // the 4 scales of combo (a, q) of group g (g < 0: zeros):
    // n = wn*WN + 32a + 8q + 4h + [0..3]
    // FAST: sr keeps the 4 fp16 scales packed (the flush's fma widens them)
    // and sv holds c = -B * s for each.
    auto read_scales = [&](int g, int combo, float (&sv)[4], uint32_t (&sr)[2])
                           __attribute__((always_inline)) {
      // the row sits in the slot of the stage the group starts in (a
      // wave-uniform choice: g < 0 reads the zero row)
      const int8_t* base = g < 0 ? smem + kZeroRow
                                 : smem + PG_RING + ((g * SUBG / 4) % PG_SNS) * PG_SSLOT +
                                       (g % SRPS) * ROWB;
      const int nl = wn * PG_WN + (combo / 4) * 32 + 8 * (combo % 4) + 4 * h;
      if constexpr (FAST) {
        const i32x2 v = *reinterpret_cast<const i32x2*>(base + nl * 2);
        sr[0] = (uint32_t)v[0];
        sr[1] = (uint32_t)v[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = __builtin_fmaf(pg_half(sr, i), -kPgBias, 0.0f);
      } else if constexpr (SWH) {
        const i32x2 v = *reinterpret_cast<const i32x2*>(base + nl * 2);
        sv[0] = h2f((uint16_t)((uint32_t)v[0] & 0xffffu));
        sv[1] = h2f((uint16_t)((uint32_t)v[0] >> 16));
        sv[2] = h2f((uint16_t)((uint32_t)v[1] & 0xffffu));
        sv[3] = h2f((uint16_t)((uint32_t)v[1] >> 16));
      } else {
        const f32x4 v = *reinterpret_cast<const f32x4*>(base + nl * 4);
        sv[0] = v[0];
        sv[1] = v[1];
        sv[2] = v[2];
        sv[3] = v[3];
      }
    };
    // Scales of the flush.  gs = 128: double-buffered by sub-step (sub-step j
    // flushes with sv[j & 1] and reads the next sub-step's into sv[(j+1) & 1]).
    // gs = 64 at two workgroups per CU (twice the combos per sub-step): one
    // buffer, read at the start of the sub-step, to save registers.
    // The fast flush's 8-wave tiles (two waves per SIMD) read them at the
    // start of the sub-step too: its scales take 6 registers per combo.
    constexpr bool SVDB = (GS == 128) || (OCC == 1 && !(FAST && NW == 8));
    float sv[SVDB ? 2 : 1][CPF][4];
    uint32_t sr[SVDB ? 2 : 1][CPF][2];  // FAST only
    auto read_sub_scales = [&](int g, int slice, int buf) __attribute__((always_inline)) {
#pragma unroll
      for (int c = 0; c < CPF; ++c) read_scales(g, slice * EPS / EPC + c, sv[buf][c], sr[buf][c]);
    };
    // t = f32(f32(D_g) * s): exact conversion and one rounding of the product,
    // or (FAST) one fma of the biased sum F = B + D_g that rounds D_g * s once
    auto term = [&](int32_t d, const float (&s)[4], const uint32_t (&r)[2], int i)
                    __attribute__((always_inline)) -> float {
      if constexpr (FAST)
        return __builtin_fmaf(__builtin_bit_cast(float, d), pg_half(r, i), s[i]);
      else
        return (float)d * s[i];
    };

    // One k sub-step J of the stage in a fixed order (sched_barrier): the
    // MFMAs into set CS (C = 0 when `first`), the next sub-step's fragment
    // reads one per MFMA in consumption order (rd) together with its flush
    // scales (group ng, slice ns), this wave's DMA loads of stage dst into slot
    // dsl (dma), and the flush of slice SL of the previous group from set
    // 1 - CS (EPM accumulators after each MFMA).
    auto step = [&](auto CSc, auto firstc, auto rdc, auto dmac, auto SLc, auto Jc,
                    const i32x4 (&wc)[PG_TN], const i32x4 (&xc)[PG_TM], int rs,
                    i32x4 (&wn_)[PG_TN], i32x4 (&xn)[PG_TM], int dst, int dsl, int ng, int ns,
                    int cg) __attribute__((always_inline)) {
      constexpr int CS = decltype(CSc)::value, SL = decltype(SLc)::value, J = decltype(Jc)::value;
      constexpr int JN = (J + 1) % 4;  // the sub-step whose operands are read
      constexpr bool first = decltype(firstc)::value != 0;
      constexpr bool rd = decltype(rdc)::value != 0;
      constexpr bool dma = decltype(dmac)::value != 0;
      if constexpr (!SVDB) read_sub_scales(cg, SL, 0);
#pragma unroll
      for (int idx = 0; idx < NMF; ++idx) {
        const int a = idx / PG_TM, b = idx % PG_TM;
        if constexpr (first)
          D[CS][a][b] = mfma32(wc[a], xc[b], cinit);
        else
          D[CS][a][b] = mfma32(wc[a], xc[b], D[CS][a][b]);
        if constexpr (rd && !W4) {
#pragma unroll
          for (int q = 0; q < NR; ++q)
            if ((q < NMF ? q : NMF - 1) == idx) {
              if (q == 0)
                read_w(rs, JN, 0, wn_);
              else if (q <= PG_TM)
                read_x(rs, JN, q - 1, xn);
              else
                read_w(rs, JN, q - PG_TM, wn_);
            }
        }
        if constexpr (rd && W4) {
          constexpr bool new_pair = (JN % 2) == 0;
          constexpr int NRD = PG_TM + (new_pair ? PG_TN : 0);
#pragma unroll
          for (int q = 0; q < NRD; ++q)
            if ((q < NMF ? q : NMF - 1) == idx) {
              if (q < PG_TM)
                read_x(rs, JN, q, xn);
              else
                read_w(rs, JN, q - PG_TM, raw);
            }
          // unpack of block a2: in the last PG_TN slots, never before the slot
          // that reads its new chunk (PG_TM + a2, clamped)
#pragma unroll
          for (int a2 = 0; a2 < PG_TN; ++a2) {
            constexpr int first_slot = new_pair ? (NMF > PG_TN ? NMF - PG_TN : 0) : 0;
            const int want =
                first_slot + a2 > PG_TM + a2 || !new_pair ? first_slot + a2 : PG_TM + a2;
            if ((want < NMF ? want : NMF - 1) == idx) unpack_half(a2, JN % 2, wn_);
          }
        }
        if constexpr (rd && SVDB) {
          if (idx == 0) read_sub_scales(ng, ns, JN & 1);
        }
        if constexpr (dma) {
#pragma unroll
          for (int d = 0; d < PG_PS; ++d)
            if (d * NMF / PG_PS == idx) dma_one(dst, dsl, d);
          if (idx == 0 && wave == 0) dma_scales(dst);
        }
#pragma unroll
        for (int e = idx * EPM; e < (idx + 1) * EPM; ++e) {
          const int eg = SL * EPS + e;  // accumulator of the set
          const int combo = eg / EPC, bb = (eg / 4) % PG_TM, rr = eg % 4;
          const int c = combo - SL * EPS / EPC;  // combo within the sub-step's scales
          const int aa = combo / 4, r = 4 * (combo % 4) + rr;
          constexpr int SB = SVDB ? (J & 1) : 0;
          if constexpr (FMA) {
            facc[aa][bb][r] = __builtin_fmaf((float)D[1 - CS][aa][bb][r], sv[SB][c][rr],
                                             facc[aa][bb][r]);
          } else {
            const float t = term(D[1 - CS][aa][bb][r], sv[SB][c], sr[SB][c], rr);
            facc[aa][bb][r] = facc[aa][bb][r] + t;
          }
          // Pins this flush element to its slot: without it the compiler sinks
          // the whole flush of a group below the next group's MFMAs, in one
          // VALU block that the MFMAs no longer hide (and, at 64 x 64 waves,
          // with both versions of the set alive at once).
          asm volatile("" : "+v"(facc[aa][bb][r]));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    auto wait_stage = [&]() __attribute__((always_inline)) {
      if (wave == 0)
        wait_vmcnt<(PG_NS - 2) * (PG_PS + 1)>();
      else
        wait_vmcnt<(PG_NS - 2) * PG_PS>();
    };

    i32x4 wf[2][PG_TN], xf[2][PG_TM];
    // The zero row of the flush before the first group (read after the
    // prologue's barrier).
    if (tid < ROWB / 16) *reinterpret_cast<i32x4*>(smem + kZeroRow + tid * 16) = i32x4{0, 0, 0, 0};
    // Prologue: stages 0 .. NS-1 (a stage past the end reloads stage nk-1 into
    // a slot nobody reads, so every stage issue moves the same loads).
#pragma unroll
    for (int st = 0; st < PG_NS; ++st) {
      dma_stage(min(st, nk - 1), st);
      if (wave == 0) dma_scales(min(st, nk - 1));
    }
    bool tame = true;
    if constexpr (FMA) tame = pg_scales_tame<PG_BN, SWH>(p, n0, G, 64 * NW);
    if (wave == 0)
      wait_vmcnt<(PG_NS - 1) * (PG_PS + 1)>();
    else
      wait_vmcnt<(PG_NS - 1) * PG_PS>();
    if constexpr (FMA) {
      // workgroup vote in the unused upper half of the zero row's scale slot
      // (its first scale DMA comes stages later)
      static_assert(ROWB + 4 * NW <= PG_SSLOT, "vote words");
      uint32_t* vote = reinterpret_cast<uint32_t*>(smem + kZeroRow + ROWB);
      const bool wbad = __builtin_amdgcn_ballot_w64(!tame) != 0;  // every lane votes
      if (lane == 0) vote[wave] = wbad ? 1u : 0u;
      __syncthreads();
      uint32_t any = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) any |= vote[w];
      if (any) {
        wait_vmcnt<0>();  // the prologue's DMA lands before the workgroup ends
        pg_exact_tile<PG_BM, PG_BN, GS, SWH, WF>(p, m0, n0, 64 * NW, 0, KL, pp);
        return false;
      }
    } else {
      __syncthreads();
    }
#pragma unroll
    for (int b = 0; b < PG_TM; ++b) read_x(0, 0, b, xf[0]);
#pragma unroll
    for (int a = 0; a < PG_TN; ++a) {
      if constexpr (W4) {
        read_w(0, 0, a, raw);
        unpack_half(a, 0, wf[0]);
      } else {
        read_w(0, 0, a, wf[0]);
      }
    }

    if constexpr (SVDB) read_sub_scales(-1, 0, 0);  // first flush: zero sum, zero scales

    // Stage kt at position HALF (0 .. PER-1) of a PER-stage period that starts
    // at a multiple of PER, so group parities are compile-time.  Sub-step J
    // belongs to group (4 kt + J) / SUBG and flushes slice (4 HALF + J) % SUBG
    // of the group before it.  LAST: the final stage (no barrier or DMA;
    // requests sa and bias; then flushes its own last group).
    auto stage = [&](int kt, auto halfc, auto lastc) __attribute__((always_inline)) {
      constexpr int HALF = decltype(halfc)::value;
      constexpr bool LAST = decltype(lastc)::value != 0;
      const int sl = kt % PG_NS;
      if constexpr (LAST) {
        sa_t = p.sa[min(m0 + tid % PG_BM, M - 1)];
        if (p.bias) b_t = p.bias[min(n0 + tid % PG_BN, N - 1)];
      }
      // group of sub-step J of stage k: (4 k + J) / SUBG; it flushes the one before
#define PG_SUB(J)                                                                            \
    {                                                                                          \
      constexpr int S = 4 * HALF + (J);                                                        \
      constexpr int CS = (S / SUBG) & 1;                                                       \
      constexpr bool FIRST = (S % SUBG) == 0;                                                  \
      constexpr int SL = S % SUBG;                                                             \
      const int cg = (4 * kt + (J)) / SUBG - 1;                                                \
      const int ng = (4 * kt + (J) + 1) / SUBG - 1;                                            \
      if constexpr ((J) < 3) {                                                                 \
        step(ic<CS>{}, ic<FIRST>{}, ic<1>{}, ic<0>{}, ic<SL>{}, ic<(J)>{}, wf[(J) & 1],       \
             xf[(J) & 1], sl, wf[((J) + 1) & 1], xf[((J) + 1) & 1], 0, 0, ng, (S + 1) % SUBG,  \
             cg);                                                                              \
      } else if constexpr (!LAST) {                                                            \
        wait_stage();                                                                          \
        __syncthreads();                                                                       \
        step(ic<CS>{}, ic<FIRST>{}, ic<1>{}, ic<1>{}, ic<SL>{}, ic<(J)>{}, wf[1], xf[1],      \
             (kt + 1) % PG_NS, wf[0], xf[0], min(kt + PG_NS, nk - 1), sl, ng, (S + 1) % SUBG,  \
             cg);                                                                              \
      } else {                                                                                 \
        step(ic<CS>{}, ic<FIRST>{}, ic<0>{}, ic<0>{}, ic<SL>{}, ic<(J)>{}, wf[1], xf[1], 0,    \
             wf[0], xf[0], 0, 0, 0, 0, cg);                                                    \
      }                                                                                        \
    }
      PG_SUB(0)
      PG_SUB(1)
      PG_SUB(2)
      PG_SUB(3)
#undef PG_SUB
      if constexpr (LAST) {
        // flush the last group (set of sub-step 3), in order
        constexpr int CSL = ((4 * HALF + 3) / SUBG) & 1;
        const int gl = G - 1;
#pragma unroll
        for (int combo = 0; combo < NCOMBO; ++combo) {
          float s4[4];
          uint32_t r4[2];
          read_scales(gl, combo, s4, r4);
          const int aa = combo / 4, q = combo % 4;
#pragma unroll
          for (int bb = 0; bb < PG_TM; ++bb)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              if constexpr (FMA) {
                facc[aa][bb][4 * q + rr] = __builtin_fmaf((float)D[CSL][aa][bb][4 * q + rr],
                                                          s4[rr], facc[aa][bb][4 * q + rr]);
              } else {
                const float t = term(D[CSL][aa][bb][4 * q + rr], s4, r4, rr);
                facc[aa][bb][4 * q + rr] = facc[aa][bb][4 * q + rr] + t;
              }
            }
        }
      }
    };

    int kt = 0;
    if constexpr (PER == 2) {
      for (; kt + 2 < nk; kt += 2) {
        stage(kt, ic<0>{}, ic<0>{});
        stage(kt + 1, ic<1>{}, ic<0>{});
      }
      if (kt + 1 < nk) {
        stage(kt, ic<0>{}, ic<0>{});
        stage(kt + 1, ic<1>{}, ic<1>{});
      } else {
        stage(kt, ic<0>{}, ic<1>{});
      }
    } else {
      // gs 256: K % 256 == 0, so nk is even and 2 or 4 stages remain
      for (; kt + 4 < nk; kt += 4) {
        stage(kt, ic<0>{}, ic<0>{});
        stage(kt + 1, ic<1>{}, ic<0>{});
        stage(kt + 2, ic<2>{}, ic<0>{});
        stage(kt + 3, ic<3>{}, ic<0>{});
      }
      if (kt + 2 < nk) {
        stage(kt, ic<0>{}, ic<0>{});
        stage(kt + 1, ic<1>{}, ic<0>{});
        stage(kt + 2, ic<2>{}, ic<0>{});
        stage(kt + 3, ic<3>{}, ic<1>{});
      } else {
        stage(kt, ic<0>{}, ic<0>{});
        stage(kt + 1, ic<1>{}, ic<1>{});
      }
    }
    wait_vmcnt<0>();  // reloads past the end land before LDS is reused
    return true;
  };

  // the fast flush where its registers fit (int8 weights at two workgroups
  // per CU would drop to one)
  constexpr bool FASTOK = SWH && !(WF == W_I8 && OCC == 2);
  if constexpr (!SWH) {
    if (!kpass(ic<2>{})) return;  // the tile ran the exact fallback
  } else if constexpr (FASTOK) {
    kpass(ic<1>{});
    // A NaN accumulator means a scale of the tile's columns was not finite
    // (finite fp16 scales keep every fast term finite: |D * s| < 2^22 * 2^16).
    // Then the workgroup redoes the tile with the exact flush; every wave
    // takes part, since all of them feed the DMA ring.
    bool bad = false;
#pragma unroll
    for (int a = 0; a < PG_TN; ++a)
#pragma unroll
      for (int b = 0; b < PG_TM; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) bad = bad || __builtin_isnan(facc[a][b][r]);
    __shared__ uint32_t vote[NW];
    const bool wbad = __builtin_amdgcn_ballot_w64(bad) != 0;
    if (lane == 0) vote[wave] = wbad ? 1u : 0u;
    __syncthreads();
    uint32_t any = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) any |= vote[w];
    if (any) kpass(ic<0>{});
  } else {
    kpass(ic<0>{});
  }

  if (pp) {
    // split-K slice: the chain's fp32 sums, 4 consecutive columns per store
#pragma unroll
    for (int a = 0; a < PG_TN; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int b = 0; b < PG_TM; ++b) {
          const int m = m0 + wm * PG_WM + b * 32 + frow;
          const int n = n0 + wn * PG_WN + a * 32 + 8 * q + 4 * h;
          if (m < M && n < N)
            *reinterpret_cast<f32x4*>(pp + (int64_t)m * N + n) =
                f32x4{facc[a][b][4 * q], facc[a][b][4 * q + 1], facc[a][b][4 * q + 2],
                      facc[a][b][4 * q + 3]};
        }
    return;
  }
  // ---- epilogue: LDS [0, OUT) fp16 tile, then sa [BM] and bias [BN]
  float* ssa = reinterpret_cast<float*>(smem + PG_OUT);
  uint16_t* sbias = reinterpret_cast<uint16_t*>(ssa + PG_BM);
  __syncthreads();  // every wave is done with the ring
  if (tid < PG_BM) ssa[tid] = sa_t;
  if (tid < PG_BN) sbias[tid] = b_t;
  __syncthreads();
#pragma unroll
  for (int a = 0; a < PG_TN; ++a) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = wn * PG_WN + a * 32 + 8 * q + 4 * h;
      const i32x2 bb = *reinterpret_cast<const i32x2*>(sbias + nl);
      const float bv[4] = {h2f((uint16_t)((uint32_t)bb[0] & 0xffffu)),
                           h2f((uint16_t)((uint32_t)bb[0] >> 16)),
                           h2f((uint16_t)((uint32_t)bb[1] & 0xffffu)),
                           h2f((uint16_t)((uint32_t)bb[1] >> 16))};
#pragma unroll
      for (int b = 0; b < PG_TM; ++b) {
        const int ml = wm * PG_WM + b * 32 + frow;
        const float sam = ssa[ml];
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = facc[a][b][4 * q + r] * sam;
          if (p.bias) v = v + bv[r];
          o[r] = v;
        }
        *reinterpret_cast<i32x2*>(smem + ml * PG_OUT_LD + nl * 2) =
            i32x2{(int)f2h2(o[0], o[1]), (int)f2h2(o[2], o[3])};
      }
    }
  }
  __syncthreads();
  constexpr int LPR = PG_BN / 8, RPS = 64 / LPR;
  const int cl = (lane % LPR) * 8;
  const int n = n0 + cl;
#pragma unroll 4
  for (int rr = wave * RPS + lane / LPR; rr < PG_BM; rr += NW * RPS) {
    const int m = m0 + rr;
    if (m < M && n < N)
      *reinterpret_cast<i32x4*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + n) =
          *reinterpret_cast<const i32x4*>(smem + rr * PG_OUT_LD + cl * 2);
  }
}

// One group set (int8 or int4 weights) on v_mfma_i32_16x16x64_i8: 128 x 128
// tiles of four 64 x 64 waves (4 x 4 blocks of 16 x 16, 4 int32 accumulators
// per lane and block), two workgroups per CU (two waves per SIMD), the ring,
// DMA issue, scale ring and fixed sub-step order of gemm_dma_pg_kernel.  Two
// waves on one SIMD do not overlap one wave's MFMAs with the other's VALU
// work when both mix them (a microbenchmark of 4 MFMAs + 48 flush-like VALU
// ops per wave and iteration: 498 cycles per SIMD at two waves, against 244
// for the MFMAs and 302 for the VALU ops alone), so the alternating second
// set of gemm_dma_pg_kernel buys little here, and its registers are better
// spent on a wave tile twice as large: per output and group 4 bytes of LDS
// fragment reads instead of 6.
// A 128-k stage is two sub-steps of 64 k; in sub-step j lane l holds k in
// [64 j + 16 (l / 16), + 16) of row l % 16 of both operands, so a group of
// gs >= 64 never splits a sub-step (int4 weights: the 8 bytes of nibbles of
// that k range, unpacked in the last slots of the sub-step before).  Each
// group's sum D_g lives in one int32 set; the first sub-step of group g
// flushes each block's sum of group g-1 (in group order: the fma flush, or
// the exact one with FL == 0) right before the MFMA that restarts the block
// from C = 0, with scales read into registers during the sub-step before.
// Before the first group D is zero and the scales are the zero row; the last
// group is flushed after the k-loop.  The 16 x 16 x 64 form against the
// 32 x 32 x 32 one on the same pipeline (bit-identical outputs; whole linears
// under sustained load): M=4096 N=10240 K=2560 gs 128 155.4 -> 150.7 us, gs
// 64 182.0 -> 172.7 us, gs 256 137.9 -> 133.4 us; M=8192 gs 128 300.6 ->
// 290.4 us; N=2560 K=10240 gs 128 169.6 -> 161.9 us; int4 M=4096 N=12288
// K=4096 gs 128 327.8 -> 309.5 us, gs 64 386.1 -> 367.1 us.
// ks > 0: split-K.  Workgroup (t, s) runs tile t over k in [s ks, (s+1) ks)
// (whole groups and k-stages) and writes its fp32 group chain, before the
// per-token scale, to part + s M N; pg_splitk_sum_kernel adds the slices.
template <int GS, bool SWH, int WF, int FL>
__global__ __launch_bounds__(256, 2) void gemm_dma_pg16_kernel(const GemmArgs pin, int ks,
                                                               float* part) {
  static_assert(GS == 64 || GS == 128 || GS == 256, "group size");
  constexpr int BM = 128, BN = 128, WGM = 2, WGN = 2;
  using C = PgCfg<BM, BN, WF, 2, WGM, WGN>;
  constexpr bool W4 = (WF == W_I4);
  constexpr int WB = C::WB;
  constexpr int NW = C::NW, WM = C::WM, WN = C::WN;
  constexpr int TM = WM / 16, TN = WN / 16;      // 16 x 16 blocks of the wave
  constexpr int BK = C::BK, CH = C::CH, RPI = C::RPI, CHW = C::CHW, RPIW = C::RPIW;
  constexpr int WI = C::WI, XI = C::XI, PS = C::PS, W_BYTES = C::W_BYTES, STAGE = C::STAGE;
  constexpr int NS = C::NS, RING = C::RING, SSLOT = C::SSLOT, SNS = C::SNS;
  constexpr int OUT_LD = C::OUT_LD, OUT = C::OUT;
  constexpr int SUBG = GS / 64;                  // sub-steps per group (a stage has 2)
  constexpr int SRPS = SUBG < 2 ? 2 / SUBG : 1;  // scale rows a stage brings
  constexpr int PER = SUBG <= 2 ? 1 : 2;         // stages per period of group starts
  constexpr int ESZ = SWH ? 2 : 4;
  constexpr int CPR = BN * ESZ / 16, ROWB = BN * ESZ;
  constexpr int NMF = TN * TM, NR = TN + TM;
  static_assert(NR <= NMF - TN, "int4: each block unpacked in a later slot than its read");
  static_assert(CPR * 16 * SRPS <= SSLOT && 64 / CPR >= SRPS, "scale rows per stage");
  constexpr int kZeroRow = RING + (SNS - 1) * SSLOT;
  static_assert(SNS - 1 - NS >= 2 && ROWB <= SSLOT, "zero row slot");
  __shared__ __attribute__((aligned(1024))) int8_t smem[C::SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WGM, wn = wave / WGM;
  const int frow = lane & 15, fq = lane >> 4;
  // K is the row pitch; the k-loop covers KL of it (a split-K slice: the
  // operands and scales start at the slice, and the partial sums go to pp)
  GemmArgs p = pin;
  float* pp = nullptr;
  if (ks > 0) {
    const int sl = blockIdx.y;
    p.x = pin.x + (int64_t)sl * ks;
    p.w = reinterpret_cast<const int8_t*>(pin.w) + (int64_t)sl * (W4 ? ks / 2 : ks);
    p.sw = reinterpret_cast<const int8_t*>(pin.sw) + (int64_t)(sl * (ks / GS)) * pin.N * ESZ;
    pp = part + (int64_t)sl * pin.M * pin.N;
  }
  const int M = p.M, N = p.N, K = p.K;
  const int KL = ks > 0 ? ks : K;
  const int G = KL / GS, nk = KL / BK;
  int m0, n0;
  tile_coords<BM, BN>(xcd_remap(blockIdx.x, gridDim.x), M, 0, N, m0, n0);

  const int64_t ldw = W4 ? (K >> 1) : K;
  const int8_t* const wbase = reinterpret_cast<const int8_t*>(p.w) + (int64_t)n0 * ldw;
  const int8_t* const xbase = p.x + (int64_t)m0 * K;
  uint32_t woff[WI], xoff[XI];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int row = (wave * WI + i) * RPIW + lane / CHW;
    woff[i] = (uint32_t)((int64_t)(min(n0 + row, N - 1) - n0) * ldw +
                         ((lane % CHW) ^ swz<WB>(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int row = (wave * XI + i) * RPI + lane / CH;
    xoff[i] = (uint32_t)((int64_t)(min(m0 + row, M - 1) - m0) * K +
                         ((lane % CH) ^ swz<BK>(row)) * 16);
  }
  const int srow = lane / CPR;
  const int8_t* ssrc = reinterpret_cast<const int8_t*>(p.sw) +
                       (int64_t)min(n0 + (lane % CPR) * (16 / ESZ), N - 16 / ESZ) * ESZ;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem);

  auto dma_one = [&](int st, int slot, int d) __attribute__((always_inline)) {
    const uint32_t sb = lds0 + (uint32_t)(slot * STAGE);
    if (d < WI)
      dma16s(wbase + (int64_t)st * WB, woff[d < WI ? d : 0], sb + (wave * WI + d) * 1024);
    else
      dma16s(xbase + (int64_t)st * BK, xoff[d >= WI ? d - WI : 0],
             sb + W_BYTES + (wave * XI + d - WI) * 1024);
  };
  // scale rows of stage st: its groups (gs 64: two), or the group it belongs
  // to (gs 256: also on the group's second stage, whose slot is not read)
  auto dma_scales = [&](int st) __attribute__((always_inline)) {
    const int g = min(st * 2 / SUBG + srow, G - 1);
    dma16(ssrc + (int64_t)g * N * ESZ, lds0 + RING + (uint32_t)((st % SNS) * SSLOT));
  };
  auto read_x = [&](int slot, int j, int b, i32x4 (&dst)[TM]) __attribute__((always_inline)) {
    const int8_t* Xs = smem + slot * STAGE + W_BYTES;
    const int row = wm * WM + b * 16 + frow;
    dst[b] = *reinterpret_cast<const i32x4*>(Xs + row * BK + (((4 * j + fq) ^ swz<BK>(row)) << 4));
  };
  // int8: fragment of W block a for sub-step j;  int4: its 8 bytes of nibbles
  // (raw), unpacked by unpack_w
  auto read_w = [&](int slot, int j, int a, i32x4 (&dst)[TN]) __attribute__((always_inline)) {
    const int8_t* Ws = smem + slot * STAGE;
    const int row = wn * WN + a * 16 + frow;
    dst[a] = *reinterpret_cast<const i32x4*>(Ws + row * BK + (((4 * j + fq) ^ swz<BK>(row)) << 4));
  };
  i32x2 raw[TN];
  auto read_w4 = [&](int slot, int j, int a) __attribute__((always_inline)) {
    const int8_t* Ws = smem + slot * STAGE;
    const int row = wn * WN + a * 16 + frow;
    const int c = 2 * j + (fq >> 1);
    raw[a] = *reinterpret_cast<const i32x2*>(Ws + row * WB + ((c ^ swz<WB>(row)) << 4) +
                                             8 * (fq & 1));
  };
  auto unpack_w = [&](int a, i32x4 (&dst)[TN]) __attribute__((always_inline)) {
    dst[a] = pg_unpack_w4_8((uint32_t)raw[a][0], (uint32_t)raw[a][1]);
  };
  auto read_wk = [&](int slot, int j, int a, i32x4 (&dst)[TN]) __attribute__((always_inline)) {
    if constexpr (W4)
      read_w4(slot, j, a);
    else
      read_w(slot, j, a, dst);
  };
  // the 4 scales of group g (g < 0: the zero row) for n-block a:
  // n = wn*WN + 16a + 4fq + [0..3]
  auto read_scales = [&](int g, int a, float (&s4)[4]) __attribute__((always_inline)) {
    const int8_t* base = g < 0 ? smem + kZeroRow
                               : smem + RING + ((g * SUBG / 2) % SNS) * SSLOT + (g % SRPS) * ROWB;
    const int nl = wn * WN + a * 16 + 4 * fq;
    if constexpr (SWH) {
      const i32x2 v = *reinterpret_cast<const i32x2*>(base + nl * 2);
      s4[0] = h2f((uint16_t)((uint32_t)v[0] & 0xffffu));
      s4[1] = h2f((uint16_t)((uint32_t)v[0] >> 16));
      s4[2] = h2f((uint16_t)((uint32_t)v[1] & 0xffffu));
      s4[3] = h2f((uint16_t)((uint32_t)v[1] >> 16));
    } else {
      const f32x4 v = *reinterpret_cast<const f32x4*>(base + nl * 4);
      s4[0] = v[0];
      s4[1] = v[1];
      s4[2] = v[2];
      s4[3] = v[3];
    }
  };

  float facc[TN][TM][4];
  const i32x4 zero4 = {0, 0, 0, 0};
  // the scales of the next flush, read one sub-step ahead
  float svp[TN][4];
  auto prefetch = [&](int g) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < TN; ++a) read_scales(g, a, svp[a]);
  };
  auto wait_stage = [&]() __attribute__((always_inline)) {
    if (wave == 0)
      wait_vmcnt<(NS - 2) * (PS + 1)>();
    else
      wait_vmcnt<(NS - 2) * PS>();
  };

  i32x4 wf[2][TN], xf[2][TM];
  if (tid < ROWB / 16) *reinterpret_cast<i32x4*>(smem + kZeroRow + tid * 16) = i32x4{0, 0, 0, 0};
  // Prologue: stages 0 .. NS-1 (a stage past the end reloads stage nk-1 into
  // a slot nobody reads, so every stage issue moves the same loads).
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int s2 = min(st, nk - 1);
    const uint32_t sb = lds0 + (uint32_t)(st * STAGE);
#pragma unroll
    for (int i = 0; i < WI; ++i) dma16s(wbase + (int64_t)s2 * WB, woff[i], sb + (wave * WI + i) * 1024);
#pragma unroll
    for (int i = 0; i < XI; ++i)
      dma16s(xbase + (int64_t)s2 * BK, xoff[i], sb + W_BYTES + (wave * XI + i) * 1024);
    if (wave == 0) dma_scales(s2);
  }
  bool tame = true;
  if constexpr (FL == 1) tame = pg_scales_tame<BN, SWH>(p, n0, G, 64 * NW);
  if (wave == 0)
    wait_vmcnt<(NS - 1) * (PS + 1)>();
  else
    wait_vmcnt<(NS - 1) * PS>();
  bool fma_tile = false;
  if constexpr (FL == 1) {
    static_assert(ROWB + 4 * NW <= SSLOT, "vote words");
    uint32_t* vote = reinterpret_cast<uint32_t*>(smem + kZeroRow + ROWB);
    const bool wbad = __builtin_amdgcn_ballot_w64(!tame) != 0;
    if (lane == 0) vote[wave] = wbad ? 1u : 0u;
    __syncthreads();
    uint32_t any = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) any |= vote[w];
    fma_tile = any == 0;
  } else {
    __syncthreads();
  }
  float sa_t = 0.0f;
  uint16_t b_t = 0;
  auto body = [&](auto fmac) __attribute__((always_inline)) {
    constexpr bool FMA = decltype(fmac)::value != 0;
    i32x4 D[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        D[a][b] = zero4;
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[a][b][r] = 0.0f;
      }
    // flush of block (a, b), each element pinned after its update so the
    // compiler keeps the conversions next to their use
    auto flush_blk = [&](int a, int b) __attribute__((always_inline)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (FMA) {
          facc[a][b][r] = __builtin_fmaf((float)D[a][b][r], svp[a][r], facc[a][b][r]);
        } else {
          const float t = (float)D[a][b][r] * svp[a][r];
          facc[a][b][r] = facc[a][b][r] + t;
        }
        asm volatile("" : "+v"(facc[a][b][r]));
      }
    };
    // One 64-k sub-step in a fixed order: per MFMA slot (block a, b), the
    // flush of the block's previous group (first sub-step of a group), the
    // MFMA, one of the next sub-step's fragment reads (rd) and a share of the
    // DMA loads of stage dst into slot dsl (dma); before a sub-step that
    // flushes (pre), the scales of group pg after the first MFMA.
    auto step = [&](auto firstc, auto rdc, auto dmac, auto JNc, auto prec, const i32x4 (&wc)[TN],
                    const i32x4 (&xc)[TM], int rs, i32x4 (&wn_)[TN], i32x4 (&xn)[TM], int dst,
                    int dsl, int pg) __attribute__((always_inline)) {
      constexpr bool first = decltype(firstc)::value != 0;
      constexpr bool pre = decltype(prec)::value != 0;
      constexpr bool rd = decltype(rdc)::value != 0;
      constexpr bool dma = decltype(dmac)::value != 0;
      constexpr int JN = decltype(JNc)::value;
#pragma unroll
      for (int idx = 0; idx < NMF; ++idx) {
        const int a = idx / TM, b = idx % TM;
        if constexpr (first) {
          flush_blk(a, b);
          D[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wc[a], xc[b], zero4, 0, 0, 0);
        } else {
          D[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wc[a], xc[b], D[a][b], 0, 0, 0);
        }
        if constexpr (rd) {
#pragma unroll
          for (int q = 0; q < NR; ++q)
            if (q == idx) {
              if (q == 0)
                read_wk(rs, JN, 0, wn_);
              else if (q <= TM)
                read_x(rs, JN, q - 1, xn);
              else
                read_wk(rs, JN, q - TM, wn_);
            }
          // int4: block a's nibbles, read in slot 0 or TM + a, unpacked in
          // slot NMF - TN + a
          if constexpr (W4) {
#pragma unroll
            for (int a2 = 0; a2 < TN; ++a2)
              if (NMF - TN + a2 == idx) unpack_w(a2, wn_);
          }
        }
        if constexpr (dma) {
#pragma unroll
          for (int d = 0; d < PS; ++d)
            if (d * NMF / PS == idx) dma_one(dst, dsl, d);
          if (idx == 0 && wave == 0) dma_scales(dst);
        }
        if constexpr (pre) {
          if (idx == NMF - 1) prefetch(pg);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
#pragma unroll
    for (int b = 0; b < TM; ++b) read_x(0, 0, b, xf[0]);
#pragma unroll
    for (int a = 0; a < TN; ++a) {
      read_wk(0, 0, a, wf[0]);
      if constexpr (W4) unpack_w(a, wf[0]);
    }
    prefetch(-1);  // the first flush: zero sums, zero scales

    // Stage kt at position HALF of a PER-stage period: sub-step J starts group
    // (2 kt + J) / SUBG when (2 HALF + J) % SUBG == 0, flushing the group
    // before; the sub-step before it reads that group's scales (PRE).
    auto stage = [&](int kt, auto halfc, auto lastc) __attribute__((always_inline)) {
      constexpr int HALF = decltype(halfc)::value;
      constexpr bool LAST = decltype(lastc)::value != 0;
      const int sl = kt % NS;
      if constexpr (LAST) {
        sa_t = p.sa[min(m0 + tid % BM, M - 1)];
        if (p.bias) b_t = p.bias[min(n0 + tid % BN, N - 1)];
      }
      {
        constexpr bool FIRST = ((2 * HALF) % SUBG) == 0;
        constexpr bool PRE = ((2 * HALF + 1) % SUBG) == 0;
        const int pg = (2 * kt + 1) / SUBG - 1;
        step(ic<FIRST>{}, ic<1>{}, ic<0>{}, ic<1>{}, ic<PRE>{}, wf[0], xf[0], sl, wf[1], xf[1], 0,
             0, pg);
      }
      {
        constexpr bool FIRST = ((2 * HALF + 1) % SUBG) == 0;
        constexpr bool PRE = ((2 * HALF + 2) % SUBG) == 0;
        const int pg = (2 * kt + 2) / SUBG - 1;
        if constexpr (!LAST) {
          wait_stage();
          __syncthreads();
          step(ic<FIRST>{}, ic<1>{}, ic<1>{}, ic<0>{}, ic<PRE>{}, wf[1], xf[1], (kt + 1) % NS,
               wf[0], xf[0], min(kt + NS, nk - 1), sl, pg);
        } else {
          step(ic<FIRST>{}, ic<0>{}, ic<0>{}, ic<0>{}, ic<PRE>{}, wf[1], xf[1], 0, wf[0], xf[0],
               0, 0, pg);
        }
      }
    };
    int kt = 0;
    if constexpr (PER == 1) {
      for (; kt + 1 < nk; ++kt) stage(kt, ic<0>{}, ic<0>{});
      stage(kt, ic<0>{}, ic<1>{});
    } else {
      // gs 256: K % 256 == 0, so nk is even
      for (; kt + 2 < nk; kt += 2) {
        stage(kt, ic<0>{}, ic<0>{});
        stage(kt + 1, ic<1>{}, ic<0>{});
      }
      stage(kt, ic<0>{}, ic<0>{});
      stage(kt + 1, ic<1>{}, ic<1>{});
    }
    // the last group (its scales were read in the last sub-step)
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b) flush_blk(a, b);
  };
  // ---- epilogue: LDS [0, OUT) fp16 tile, then sa [BM] and bias [BN]
  auto epilogue = [&]() __attribute__((always_inline)) {
    wait_vmcnt<0>();  // reloads past the end land before LDS is reused
    float* ssa = reinterpret_cast<float*>(smem + OUT);
    uint16_t* sbias = reinterpret_cast<uint16_t*>(ssa + BM);
    __syncthreads();  // every wave is done with the ring
    if (tid < BM) ssa[tid] = sa_t;
    if (tid < BN) sbias[tid] = b_t;
    __syncthreads();
#pragma unroll
    for (int a = 0; a < TN; ++a) {
      const int nl = wn * WN + a * 16 + 4 * fq;
      const i32x2 bb = *reinterpret_cast<const i32x2*>(sbias + nl);
      const float bv[4] = {h2f((uint16_t)((uint32_t)bb[0] & 0xffffu)),
                           h2f((uint16_t)((uint32_t)bb[0] >> 16)),
                           h2f((uint16_t)((uint32_t)bb[1] & 0xffffu)),
                           h2f((uint16_t)((uint32_t)bb[1] >> 16))};
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int ml = wm * WM + b * 16 + frow;
        const float sam = ssa[ml];
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = facc[a][b][r] * sam;
          if (p.bias) v = v + bv[r];
          o[r] = v;
        }
        *reinterpret_cast<i32x2*>(smem + ml * OUT_LD + nl * 2) =
            i32x2{(int)f2h2(o[0], o[1]), (int)f2h2(o[2], o[3])};
      }
    }
    __syncthreads();
    constexpr int LPR = BN / 8, RPS = 64 / LPR;
    const int cl = (lane % LPR) * 8;
    const int n = n0 + cl;
#pragma unroll 4
    for (int rr = wave * RPS + lane / LPR; rr < BM; rr += NW * RPS) {
      const int m = m0 + rr;
      if (m < M && n < N)
        *reinterpret_cast<i32x4*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + n) =
            *reinterpret_cast<const i32x4*>(smem + rr * OUT_LD + cl * 2);
    }
  };
  // split-K slice: the chain's fp32 sums, 4 consecutive columns per store
  auto store_part = [&]() __attribute__((always_inline)) {
    wait_vmcnt<0>();  // reloads past the end land before the workgroup ends
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int m = m0 + wm * WM + b * 16 + frow;
        const int n = n0 + wn * WN + a * 16 + 4 * fq;
        if (m < M && n < N)
          *reinterpret_cast<f32x4*>(pp + (int64_t)m * N + n) =
              f32x4{facc[a][b][0], facc[a][b][1], facc[a][b][2], facc[a][b][3]};
      }
  };
  if constexpr (FL == 1) {
    if (fma_tile) {
      body(ic<1>{});
      if (pp)
        store_part();
      else
        epilogue();
    } else {
      wait_vmcnt<0>();  // the prologue's DMA lands before the workgroup ends
      pg_exact_tile<BM, BN, GS, SWH, WF>(p, m0, n0, 64 * NW, 0, KL, pp);
    }
  } else {
    body(ic<0>{});
    if (pp)
      store_part();
    else
      epilogue();
  }
}

// Eligible: int8 or int4 weights, per-group gs 64 / 128 (gs 256: int8 and
// K % 256 == 0), K % 128 == 0, N % 8 == 0, 16-byte aligned operands
// (launch_gemm checks).
namespace {

// 64 x 64 tiles of four 32 x 32 waves, for grids the larger tiles leave
// mostly idle.
template <int GS, bool SWH, int WF>
hipError_t run_pg64(const GemmArgs& a, hipStream_t s) {
  const int tiles = ((a.M + 63) / 64) * ((a.N + 63) / 64);
  gemm_dma_pg_kernel<64, 64, GS, SWH, WF, 2, 2, 2><<<tiles, 256, 0, s>>>(a, 0, nullptr);
  return hipGetLastError();
}

}  // namespace

// y[m, n..n+3] = h(f32((sum over s of part[s][m][n], in slice order) * sa[m])
// [+ bias[n]]); N % 4 == 0, so a thread's four columns share a row.
__global__ __launch_bounds__(256) void pg_splitk_sum_kernel(const GemmArgs p,
                                                            const float* __restrict__ part,
                                                            int S) {
  const int64_t MN = (int64_t)p.M * p.N;
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= MN) return;
  const int m = (int)(e / p.N), n = (int)(e % p.N);
  f32x4 acc = *reinterpret_cast<const f32x4*>(part + e);
  for (int sl = 1; sl < S; ++sl) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(part + sl * MN + e);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = acc[r] + v[r];
  }
  const float sam = p.sa[m];
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = acc[r] * sam;
    if (p.bias) v = v + h2f(p.bias[n + r]);
    o[r] = v;
  }
  *reinterpret_cast<i32x2*>(reinterpret_cast<uint16_t*>(p.y) + e) =
      i32x2{(int)f2h2(o[0], o[1]), (int)f2h2(o[2], o[3])};
}

// Tile of the split-K slices, with the workgroups one CU holds and the
// shortest slice: 128 x 128 (eight 64 x 32 waves, one per CU, 2048 k) from
// 256 rows; below that 128 x 64 (four 64 x 32 waves, two per CU, 2048 k), and
// for gs 256 64 x 64 (four 32 x 32 waves, two per CU, 1024 k: 27.5 against
// 29.7 us for 128 x 128 at M=128 N=2560 K=10240).
namespace {
struct PgSplitTile {
  int bm, bn, per_cu, min_slice;
};
PgSplitTile pg_split_tile(int M, int gs) {
  if (M >= 256) return {128, 128, 1, 2048};
  if (gs == 256) return {64, 64, 2, 1024};
  return {128, 64, 2, 2048};
}

// Slices of the two-set kernel: the most, in powers of two up to 8, that keep
// the slices' workgroups within what the CUs hold at once, each slice of
// whole groups and no shorter than the tile's minimum.  Measured (kernels +
// slice sum, weights from HBM, against the 64 x 64 tiles in up to eight
// slices within two workgroups per CU that ran before, and the unsplit
// dispatch at M >= 256): int8 M=128 N=2560 K=10240 gs 64 23.1 -> 21.6 us,
// gs 128 22.3 -> 19.7 us; M=256 gs 64 37.8 -> 27.0 us, gs 128 30.2 -> 25.2
// us; M=512 gs 128 42.0 -> 36.1 us; int4 M=512 N=4096 K=12288 gs 128 65.5 ->
// 55.4 us, gs 64 84.8 -> 68.6 us; M=128 gs 128 25.7 -> 24.6 us.  Grids that
// already fill the CUs, or short K (M=128 N=10240 K=2560: 16.8 against 20.0
// us in two slices), do not split.  The slices' fp32 chains are added in
// slice order, so the result follows the per-group tolerance bar, not the
// sequential chain's bits.  The caller checks the DMA conditions
// (K % 128 == 0, N % 8 == 0, aligned operands, K * 256 < 2^32).
int pg_splitk_ways_two_set(int M, int N, int K, int gs) {
  const PgSplitTile t = pg_split_tile(M, gs);
  const int slots = t.per_cu * num_cus();
  const int tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  const int unit = gs > 128 ? gs : 128;
  int S = 1;
  while (S < 8 && tiles * 2 * S <= slots && K % (unit * 2 * S) == 0 &&
         K / (2 * S) >= t.min_slice)
    S *= 2;
  return S;
}

struct PgSplit {
  int S;         // K slices (1: no split)
  bool one_set;  // slices of gemm_dma_pg16_kernel, else of gemm_dma_pg_kernel
};

// K slices of the per-group linear (1 = no split) at M > 64 (smaller M runs
// the skinny kernels), and whether the one-set kernel runs them.  Grids of
// the one-set kernel's 128 x 128 tiles that fill one and a half of its two
// workgroups per CU run unsplit.  Below that, its slices where the most of
// them (powers of two up to 8, within two workgroups per CU, at least 1024 k
// each, whole groups) fill one and a half workgroups per CU again: W4A8 M=512
// N=4096 K=12288 gs 64 75.9 -> 68.1 us, gs 128 61.0 -> 59.4 us (four slices
// against two of the two-set kernel).  With fewer of its slices the one-set
// kernel lost (int8 gs 64 M=1024 N=2560 K=10240: 76.0 against 69.9 us
// unsplit; M=128 N=2560 K=10240 gs 128: 26.5 against 24.8 us), so the other
// shapes keep the two-set kernel's slices above.
PgSplit pg_split_plan(int M, int N, int K, int gs) {
  if (M <= 64 || N % 8 != 0 || K % 128 != 0) return {1, false};
  if ((int64_t)K * 256 >= ((int64_t)1 << 32)) return {1, false};
  const int cus = num_cus();
  const int tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (2 * tiles >= 3 * cus) return {1, false};
  const int unit = gs > 128 ? gs : 128;
  int S = 1;
  while (S < 8 && tiles * 2 * S <= 2 * cus && K % (unit * 2 * S) == 0 && K / (2 * S) >= 1024)
    S *= 2;
  if (S > 1 && 2 * tiles * S >= 3 * cus) return {S, true};
  return {pg_splitk_ways_two_set(M, N, K, gs), false};
}

}  // namespace

int pg_splitk_ways(int M, int N, int K, int gs) { return pg_split_plan(M, N, K, gs).S; }

size_t pg_splitk_bytes(int M, int N, int K, int gs) {
  const int S = pg_splitk_ways(M, N, K, gs);
  return S > 1 ? (size_t)S * M * N * 4 : 0;
}

namespace {

template <int GS, bool SWH, int WF>
hipError_t run_pg_splitk(const GemmArgs& a, int S, float* part, hipStream_t s) {
  if constexpr (!(WF == W_I4 && GS == 256)) {
    if (pg_split_plan(a.M, a.N, a.K, GS).one_set) {
      const dim3 grid(((a.M + 127) / 128) * ((a.N + 127) / 128), S);
      gemm_dma_pg16_kernel<GS, SWH, WF, 1><<<grid, 256, 0, s>>>(a, a.K / S, part);
      return hipGetLastError();
    }
  }
  const PgSplitTile t = pg_split_tile(a.M, GS);
  const int bm = t.bm, bn = t.bn;
  const dim3 grid(((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn), S);
  if (bn == 128) {
    gemm_dma_pg_kernel<128, 128, GS, SWH, WF, 1, 2, 4><<<grid, 512, 0, s>>>(a, a.K / S, part);
  } else if (bm == 64) {
    gemm_dma_pg_kernel<64, 64, GS, SWH, WF, 2, 2, 2><<<grid, 256, 0, s>>>(a, a.K / S, part);
  } else {
    if constexpr (GS != 256)
      gemm_dma_pg_kernel<128, 64, GS, SWH, WF, 2, 2, 2><<<grid, 256, 0, s>>>(a, a.K / S, part);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_pg_splitk(const GemmArgs& a, int gs, bool sw_half, int wf, int S,
                                 float* part, hipStream_t s) {
  hipError_t e;
  if (wf == W_I4)
    e = gs == 64 ? run_pg_splitk<64, true, W_I4>(a, S, part, s)
                 : run_pg_splitk<128, true, W_I4>(a, S, part, s);
  else if (sw_half)
    e = gs == 64 ? run_pg_splitk<64, true, W_I8>(a, S, part, s)
        : gs == 128 ? run_pg_splitk<128, true, W_I8>(a, S, part, s)
                    : run_pg_splitk<256, true, W_I8>(a, S, part, s);
  else
    e = gs == 64 ? run_pg_splitk<64, false, W_I8>(a, S, part, s)
        : gs == 128 ? run_pg_splitk<128, false, W_I8>(a, S, part, s)
                    : run_pg_splitk<256, false, W_I8>(a, S, part, s);
  if (e != hipSuccess) return e;
  const int64_t quads = ((int64_t)a.M * a.N) / 4;
  pg_splitk_sum_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, s>>>(a, part, S);
  return hipGetLastError();
}

hipError_t launch_gemm_dma_pg(const GemmArgs& a, int gs, bool sw_half, int wf, hipStream_t s) {
  {
    // Mid M on small N: when the tiles below would fill at most half the
    // CUs, 64 x 64 tiles give four times as many workgroups (the group chain
    // rules out splitting K across workgroups).  Weights from HBM: gs 128
    // M=128 N=2560 K=10240 48.9 -> 35.3 us, gs 64 M=512 N=4096 K=12288 99.0
    // -> 77.4 us; at twice that many large tiles the 64 x 64 grid was slower.
    const int big = gs == 128 ? ((a.M + 127) / 128) * ((a.N + 63) / 64)
                              : ((a.M + 127) / 128) * ((a.N + 127) / 128);
    if (2 * big <= num_cus()) {
      if (wf == W_I4) return gs == 64 ? run_pg64<64, true, W_I4>(a, s) : run_pg64<128, true, W_I4>(a, s);
      if (sw_half) {
        if (gs == 64) return run_pg64<64, true, W_I8>(a, s);
        if (gs == 128) return run_pg64<128, true, W_I8>(a, s);
        return run_pg64<256, true, W_I8>(a, s);
      }
      if (gs == 64) return run_pg64<64, false, W_I8>(a, s);
      if (gs == 128) return run_pg64<128, false, W_I8>(a, s);
      return run_pg64<256, false, W_I8>(a, s);
    }
  }
  {
    // The one-set kernel: 128 x 128 tiles of four 64 x 64 waves, two
    // workgroups per CU, for int8 weights with fp32 scales and int4 weights
    // with fp16 scales, once its tiles fill 384 of the 512 workgroup slots
    // (the fma chain of the kernels below for fp32 scales; from 384 instead
    // of 512: W4A8 gs 64 M=512 N=12288 K=4096 87.8 -> 71.6 us, gs 128 60.2
    // -> 58.8 us).  Against the two-set
    // kernel's tiles, measured on its 32 x 32 x 32 form (the 16 x 16 x 64
    // form it runs now is 3-6 % faster again; weights from HBM where they
    // exceed the MALL): M=4096 N=10240 K=2560 gs
    // 128 188.5 -> 153.9 us, gs 64 228.8 -> 197.4 us, gs 256 163.2 -> 136.5
    // us; M=4096 N=2560 K=10240 gs 128 171.1 -> 159.1 us; M=1024 N=10240
    // K=2560 gs 128 49.4 -> 46.7 us; M=2048 95.3 -> 79.7 us; int4 M=4096
    // N=12288 K=4096 gs 128 368.8 -> 337.3 us, gs 64 478.4 -> 430.0 us; int4
    // M=1024 N=12288 K=4096 gs 128 95.9 -> 90.5 us.  256 x 128 tiles of 8
    // waves (one workgroup per CU) ran level at five rounds and up to 20 %
    // slower where their grid leaves a partial round; below one round of
    // 128 x 128 tiles the two-set kernel stayed ahead on some shapes (int4
    // M=512 N=12288 K=4096 gs 128: 52.3 against 55.8 us).
    const int64_t tiles = (int64_t)((a.M + 127) / 128) * ((a.N + 127) / 128);
    const bool fmt = (wf == W_I8 && !sw_half) || (wf == W_I4 && sw_half && gs != 256);
    if (fmt && 2 * tiles >= 3 * (int64_t)num_cus()) {
      const unsigned grid = (unsigned)tiles;
      if (wf == W_I4) {
        if (gs == 64)
          gemm_dma_pg16_kernel<64, true, W_I4, 1><<<grid, 256, 0, s>>>(a, 0, nullptr);
        else
          gemm_dma_pg16_kernel<128, true, W_I4, 1><<<grid, 256, 0, s>>>(a, 0, nullptr);
      } else if (gs == 64) {
        gemm_dma_pg16_kernel<64, false, W_I8, 1><<<grid, 256, 0, s>>>(a, 0, nullptr);
      } else if (gs == 128) {
        gemm_dma_pg16_kernel<128, false, W_I8, 1><<<grid, 256, 0, s>>>(a, 0, nullptr);
      } else {
        gemm_dma_pg16_kernel<256, false, W_I8, 1><<<grid, 256, 0, s>>>(a, 0, nullptr);
      }
      return hipGetLastError();
    }
  }
  if (gs == 256) {
    // int8 weights only (the W4A8 formats define gs 64 / 128); the 8-wave
    // 128 x 128 tile: 205.6 us at M=4096 N=10240 K=2560 against 225.8 us for
    // two 128 x 64 workgroups per CU (and 280.1 us on the register-staged
    // kernel that ran gs 256 before)
    constexpr int BM = 128, BN = 128;
    const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    if (sw_half)
      gemm_dma_pg_kernel<BM, BN, 256, true, W_I8, 1, 2, 4><<<tiles, 512, 0, s>>>(a, 0, nullptr);
    else
      gemm_dma_pg_kernel<BM, BN, 256, false, W_I8, 1, 2, 4><<<tiles, 512, 0, s>>>(a, 0, nullptr);
    return hipGetLastError();
  }
  if (gs == 64 && a.M > 64) {
    // 128 x 128 tiles, 8 waves of 64 x 32 (two per SIMD), all registers
    // architectural: 1.65x the rate of the one-wave-per-SIMD 128 x 64 tile
    // at M=4096 N=10240 K=2560 (229 vs 382 us), and ahead even where its
    // fewer tiles leave CUs idle, since each tile runs at twice the rate.
    constexpr int BM = 128, BN = 128;
    const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    if (wf == W_I4)
      gemm_dma_pg_kernel<BM, BN, 64, true, W_I4, 1, 2, 4><<<tiles, 512, 0, s>>>(a, 0, nullptr);
    else if (sw_half)
      gemm_dma_pg_kernel<BM, BN, 64, true, W_I8, 1, 2, 4><<<tiles, 512, 0, s>>>(a, 0, nullptr);
    else
      gemm_dma_pg_kernel<BM, BN, 64, false, W_I8, 1, 2, 4><<<tiles, 512, 0, s>>>(a, 0, nullptr);
    return hipGetLastError();
  }
  // 128 x 64 tiles, 4 waves of 64 x 32: gs 128 runs two workgroups per CU
  // (the 8-wave 128 x 128 tile measured level with it), gs 64 at M <= 64 one
  constexpr int BM = 128, BN = PG_LAUNCH_BN;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (wf == W_I4) {
    // int4 weights come with fp16 group scales ([K/gs, N])
    if (gs == 64)
      gemm_dma_pg_kernel<BM, BN, 64, true, W_I4, 1, 2, 2><<<tiles, 256, 0, s>>>(a, 0, nullptr);
    else
      gemm_dma_pg_kernel<BM, BN, 128, true, W_I4, 2, 2, 2><<<tiles, 256, 0, s>>>(a, 0, nullptr);
  } else if (gs == 64) {
    if (sw_half)
      gemm_dma_pg_kernel<BM, BN, 64, true, W_I8, 1, 2, 2><<<tiles, 256, 0, s>>>(a, 0, nullptr);
    else
      gemm_dma_pg_kernel<BM, BN, 64, false, W_I8, 1, 2, 2><<<tiles, 256, 0, s>>>(a, 0, nullptr);
  } else {
    if (sw_half)
      gemm_dma_pg_kernel<BM, BN, 128, true, W_I8, 2, 2, 2><<<tiles, 256, 0, s>>>(a, 0, nullptr);
    else
      gemm_dma_pg_kernel<BM, BN, 128, false, W_I8, 2, 2, 2><<<tiles, 256, 0, s>>>(a, 0, nullptr);
  }
  return hipGetLastError();
}

}  // namespace cider
