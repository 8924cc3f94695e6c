// Tiled int8 GEMM, main path for int8 weights (int32 and per-channel
// epilogues) and int4 weights (per-channel, the reference W4A8) with
// K % 128 == 0 and N % 8 == 0: operands stream global -> LDS by gfx950's
// 16-byte LDS-DMA loads through a ring of k-stages, the MFMAs are
// v_mfma_i32_32x32x32_i8, and the fp16 tile is staged through LDS so the
// output is written in whole rows.
//
// Reference semantics are those of gemm.hip (same epilogues, same fp32
// operation order, bit-identical results):
//   EPI_I32 cider/kernels/w8a8_matmul.metal:301-453
//   EPI_PC  cider/kernels/w8a8_matmul.metal:63-81
//   int4    cider/kernels/w4a8_matmul.metal:47-89,189-246 (no bias)
// (Per-group gs 64 / 128 runs gemm_dma_pg.hip, which brings the group scales
// in by LDS-DMA too: a compiler-visible scale load in the k-loop would make
// the compiler wait for every LDS-DMA load in flight.  gs 256 and shapes this
// kernel does not take run the register-staged kernel of gemm.hip.)
//
// MI355X design
//   * One workgroup per CU; tile BM (m) x BN (n) from {256 x 256, 192 x 256,
//     128 x 256, 128 x 128, 128 x 64, 64 x 128, 64 x 64}, picked per shape by
//     measured rate and the rounds the grid needs on the 256 CUs.  Waves: 2
//     along m and NWV / 2 along n.  The 256-column tiles run NWV = 8 waves,
//     two per SIMD: at 256 x 256 each wave owns 128 x 64 = 4 x 2 blocks of
//     32 x 32 (16 int32 accumulators per lane per block, 128 registers), and
//     while one wave of a SIMD waits on its DMA issue, fragment reads or
//     epilogue, the other's MFMAs run.  That costs 1.5x the fragment reads of
//     four 128 x 128 waves (LDS ~126 B/clk per CU at the full MFMA rate,
//     against ~128 delivered) and measured faster anyway: uniform 256 x 256 at
//     M=4096 N=10240 K=2560 113.8 -> 105.9 us, the mixed grid 104.4 -> 99.8
//     us, M=8192 199.6 -> 188.0 us, int4 N=12288 K=4096 199.9 -> 190.3 us;
//     192 x 256 and 128 x 256 4-10 %; N=2560 K=10240 level.  The smaller
//     tiles keep four waves (2 x 2).  Weights are the MFMA A operand,
//     activations the B operand.  A spill reload is a vector-memory load, and
//     waiting for it waits for every DMA load in flight (one spilled build ran
//     15 % slower).
//   * K advances BK bytes per stage (128; 64 is kept for tuning); stage s
//     lives in ring slot s % NS, NS = as many stages as fit the 160 KB LDS
//     (2 at 256 x 256 x 128, 3 at 128 x 256, up to 8 for small tiles).  Each
//     wave moves its share of a stage with global_load_lds_dwordx4 (one
//     instruction = 1 KB, written contiguously to LDS at M0): no VGPR
//     staging, no ds_write.  The
//     loads are issued from inline asm, so the compiler does not wait for
//     them; every issue moves the same number of loads (a stage past the end
//     reloads the last stage into a slot nobody reads), so the wait before
//     each barrier is one constant s_waitcnt vmcnt.
//   * A stage is BK / 32 k sub-steps of TN x TM MFMAs.  Each sub-step is one
//     fixed instruction order (sched_barrier): MFMAs, with the next
//     sub-step's fragment reads issued one per MFMA in the order they will be
//     consumed, and this wave's share of DMA loads spread over the MFMAs.
//     Left to itself, the compiler regroups the reads next to the MFMAs that
//     consume them and exposes LDS latency at every sub-step.
//   * With three or more ring slots, a stage's DMA loads are spread over
//     SUBS sub-steps (the last of stage kt and the first ones of stage kt+1)
//     instead of one: the CU's vector-memory path accepts one 1 KB load per
//     ~23 cycles, and a whole stage's loads inside one sub-step stalled the
//     issuing waves for ~440 of its 512 MFMA cycles (measured at 256 x 256).
//     Two slots (int8 256 x 256) split a stage in two parts only: the second
//     part, issued in the first sub-step of stage kt+1, must land by that
//     stage's barrier.  int4 weights at 256 x 256 (three slots) issue a
//     stage whole: 4 parts measured 25-40 % slower, 2 parts level.
//   * The one barrier per stage sits before its last sub-step: it publishes
//     stage kt + 1 and frees the slot of stage kt, which then receives stage
//     kt + NS.
//   * LDS rows are BK bytes; chunk c of row r is stored in slot
//     c ^ ((r / (256 / BK)) % (BK / 16)): the 16 lanes LDS serves together
//     read 16 consecutive rows at one chunk, and land in 16 distinct 16-byte
//     bank groups.  The DMA destination is contiguous, so each lane picks the
//     global chunk of the slot it writes.
//   * Epilogue (per-channel): the tile's sw, sa and bias are requested at the
//     start of the last stage and staged in LDS; each wave reads the column
//     scales it needs into registers, then dequantizes its accumulators to
//     fp16 into a BM x BN LDS tile (rows padded by 16 bytes),
//     then the workgroup stores whole 2*BN-byte rows with 16-byte lanes, so
//     HBM sees full 128-byte lines instead of 32-byte row fragments.
//   * int4 weights: a k-stage of a weight row is 64 bytes of nibbles (the ring
//     then holds 3 stages at 256 x 256).  One ds_read_b128 per W block brings
//     the 32 nibbles of a pair of sub-steps; each sub-step's 16 are unpacked
//     to int8 in registers (sign extension by xor/sub, byte permute) one
//     sub-step ahead of their MFMAs.  The k mapping of a pair puts lane half h
//     on k 64p + 32h + [0, 32), identically for both operands, so the int32
//     dot products are exact.
//   * Rows past M or N are loaded from the last valid row (their results are
//     never stored); K % 128 == 0 is required, so there is no K tail.
#include "common.hpp"
#include "dma_common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace cider {

namespace {


template <int BM, int BN, int BK, int WF = W_I8, int NWV = 4>
struct DmaCfg {
  static constexpr int CH = BK / 16;                // 16-byte chunks per X row
  static constexpr int RPI = 1024 / BK;             // X rows per DMA instruction
  static constexpr int WB = (WF == W_I4) ? BK / 2 : BK;  // weight bytes per row and stage
  static constexpr int CHW = WB / 16;               // 16-byte chunks per W row
  static constexpr int RPIW = 1024 / WB;            // W rows per DMA instruction
  static constexpr int WI = BN / RPIW / NWV, XI = BM / RPI / NWV;  // per wave
  static constexpr int PS = WI + XI;                // vmcnt units per stage
  static constexpr int SUBS = BK / 32;              // MFMA k sub-steps per stage
  static constexpr int W_BYTES = BN * WB, X_BYTES = BM * BK, STAGE = W_BYTES + X_BYTES;
  static constexpr int NS0 = kLdsBytes / STAGE;
  static constexpr int NS = NS0 > 8 ? 8 : NS0;      // ring slots
  static constexpr int RING = NS * STAGE;
  static constexpr int OUT_LD = BN * 2 + 16;        // fp16 tile row pitch
  static constexpr int OUT = BM * OUT_LD;
  static constexpr int SCL = BN * 4 + BM * 4 + BN * 2;  // sw, sa, bias of the tile
  static constexpr int EPI_BYTES = OUT + SCL;
  static constexpr int SMEM = RING > EPI_BYTES ? RING : EPI_BYTES;
  static_assert(WI >= 1 && XI >= 1, "tile too small for the DMA split");
  static_assert(NS >= 2, "ring needs two slots");
  static_assert(SMEM <= kLdsBytes, "LDS budget");
  static_assert((NS - 2) * PS <= 63 && (NS - 1) * PS <= 63, "vmcnt range");
};

// 8 bytes of packed int4 (element 2i in the low nibble of byte i) -> 16 int8
// in element order.
__device__ __forceinline__ i32x4 unpack_w4_8(uint32_t w0, uint32_t w1) {
  uint32_t a, b, c, d;
  unpack_w4_word(w0, a, b);
  unpack_w4_word(w1, c, d);
  return i32x4{(int)a, (int)b, (int)c, (int)d};
}

template <int V>
using icst = std::integral_constant<int, V>;

}  // namespace

// One BM x BN output tile over the whole K.  smem: DmaCfg::SMEM bytes of LDS.
// WF = W_I8: weights int8 [N, K]; W_I4: packed int4 [N, K/2] (element k in
// byte k/2, low nibble first, two's complement), unpacked in registers.
template <int BM, int BN, int BK, int EPI, int WF = W_I8, int NWV = 4>
__device__ __forceinline__ void dma_tile(const GemmArgs& p, const int m0, const int n0,
                                         int8_t* __restrict__ smem, const int kloop = 0) {
  static_assert((BM == 64 || BM == 128 || BM == 192 || BM == 256) &&
                    (BN == 64 || BN == 128 || BN == 256),
                "tile shape");
  static_assert(BK == 64 || BK == 128, "k stage");
  static_assert(WF == W_I8 || BK == 128, "int4 weights use 128-byte k-stages");
  using C = DmaCfg<BM, BN, BK, WF, NWV>;
  constexpr bool W4 = (WF == W_I4);
  // waves: 2 along m, NWV / 2 along n
  constexpr int WM = BM / 2, WN = BN / (NWV / 2), TM = WM / 32, TN = WN / 32;
  constexpr int WI = C::WI, XI = C::XI, PS = C::PS, NS = C::NS, SUBS = C::SUBS;
  constexpr int W_BYTES = C::W_BYTES, STAGE = C::STAGE, CH = C::CH, RPI = C::RPI;
  constexpr int WB = C::WB, CHW = C::CHW, RPIW = C::RPIW;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int M = p.M, N = p.N, K = p.K;
  const int h = lane >> 5;

  // DMA: instruction i of this wave fills tile rows R0 = (wave*WI + i)*RPIW ..
  // + RPIW (X: RPI); lane l writes row R0 + l / CHW, slot l % CHW, which holds
  // global chunk slot ^ swz(row).
  // Sources: the tile's first W (X) row as a wave-uniform base, and per
  // lane and instruction a 32-bit byte offset from it (< 256 rows x K).
  const int64_t ldw = W4 ? (K >> 1) : K;
  const int8_t* const wbase = reinterpret_cast<const int8_t*>(p.w) + (int64_t)n0 * ldw;
  const int8_t* const xbase = p.x + (int64_t)m0 * K;
  uint32_t woff[WI], xoff[XI];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int row = (wave * WI + i) * RPIW + lane / CHW;
    const int n = min(n0 + row, N - 1);
    woff[i] = (uint32_t)((int64_t)(n - n0) * ldw + ((lane % CHW) ^ swz<WB>(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int row = (wave * XI + i) * RPI + lane / CH;
    const int m = min(m0 + row, M - 1);
    xoff[i] = (uint32_t)((int64_t)(m - m0) * K + ((lane % CH) ^ swz<BK>(row)) * 16);
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem);
  // DMA instruction d (0 .. PS-1) of this wave for stage st into ring slot
  // `slot`: W rows first, then X rows.
  auto dma_one = [&](int st, int slot, int d) {
    const uint32_t sb = lds0 + (uint32_t)(slot * STAGE);
    if (d < WI)
      dma16s(wbase + (int64_t)st * WB, woff[d < WI ? d : 0], sb + (wave * WI + d) * 1024);
    else
      dma16s(xbase + (int64_t)st * BK, xoff[d >= WI ? d - WI : 0],
             sb + W_BYTES + (wave * XI + d - WI) * 1024);
  };

  // k mapping of sub-step j for lane half h (the same for both operands):
  //   int8 weights: k in [32 j + 16 h, + 16)               (X chunk 2j + h)
  //   int4 weights: k in [64 (j/2) + 32 h + 16 (j%2), + 16) (X chunk
  //     4 (j/2) + 2h + j%2; W4 chunk 2 (j/2) + h holds the pair's 32 nibbles,
  //     read once per pair, half j%2 unpacked per sub-step)
  const int frow = lane & 31;
  auto x_chunk = [&](int j) { return W4 ? 4 * (j / 2) + 2 * h + (j % 2) : 2 * j + h; };
  auto read_x = [&](int slot, int j, int b, i32x4 (&xfn)[TM]) {
    const int8_t* Xs = smem + slot * STAGE + W_BYTES;
    const int row = wm * WM + b * 32 + frow;
    xfn[b] = *reinterpret_cast<const i32x4*>(Xs + row * BK + ((x_chunk(j) ^ swz<BK>(row)) << 4));
  };
  // int8: fragment of W block a for sub-step j;  int4: the raw 16-byte chunk
  // of W block a for the sub-step pair j / 2
  auto read_w = [&](int slot, int j, int a, i32x4 (&dst)[TN]) {
    const int8_t* Ws = smem + slot * STAGE;
    const int row = wn * WN + a * 32 + frow;
    const int c = W4 ? 2 * (j / 2) + h : 2 * j + h;
    dst[a] = *reinterpret_cast<const i32x4*>(Ws + row * WB + ((c ^ swz<WB>(row)) << 4));
  };
  i32x4 raw[TN];  // int4 only: packed chunks of the current sub-step pair
  auto unpack_half = [&](int a, int half, i32x4 (&dst)[TN]) {
    dst[a] = half == 0 ? unpack_w4_8((uint32_t)raw[a][0], (uint32_t)raw[a][1])
                       : unpack_w4_8((uint32_t)raw[a][2], (uint32_t)raw[a][3]);
  };

  i32x16 acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  // DMA loads of one stage are issued in DS parts: part 0 in the last
  // sub-step of stage kt (after the barrier that frees its slot), parts
  // 1 .. DS-1 in the first sub-steps of stage kt+1.  A stage's loads at once
  // (PS per wave inside one sub-step) outrun what the CU's vector-memory path
  // accepts (one 1 KB load per ~23 cycles) and stall the issuing waves.  Every
  // part is out before the next barrier, so the counts waited for are as if
  // the stage were issued at once.  With two slots (int8 256 x 256) the parts
  // issued in stage kt+1 have only the sub-steps before its barrier to land:
  // two parts measured 4-11% faster than one, four parts no faster than one.
  // Exception, measured: int4 weights at 256 x 256 (three slots) ran 25-40%
  // slower in 4 parts than whole, and level in 2.
  constexpr int DS = (W4 && BM == 256) ? 1 : NS >= 3 ? SUBS : 2;

  // One k sub-step in a fixed instruction order (sched_barrier): the TN*TM
  // MFMAs on fragments (wc, xc); between them the operands of the next
  // sub-step JN (from slot rs) when rd, and part dmac - 1 of this wave's DMA
  // loads of stage dst into slot dsl when dmac > 0.  int8: the next fragments are read one per MFMA
  // in the order they will be consumed (W0, X0 .. X(TM-1), W1 ..), each at
  // least TN*TM - TN - TM MFMAs before its use.  int4: the X fragments are
  // read first; when JN starts a new pair the raw W chunks are read next and
  // unpacked in the last TN MFMA slots, otherwise the second half of the
  // chunks already held is unpacked.  Left to itself the compiler regroups
  // the reads next to the MFMAs that consume them and exposes LDS latency.
  auto step = [&](auto JNc, auto rdc, auto dmac, const i32x4 (&wc)[TN], const i32x4 (&xc)[TM],
                  int rs, i32x4 (&wn_)[TN], i32x4 (&xn)[TM], int dst, int dsl) {
    constexpr int JN = decltype(JNc)::value;
    constexpr bool rd = decltype(rdc)::value != 0;
    constexpr int part = decltype(dmac)::value - 1;  // -1: no DMA
    constexpr int d0 = part < 0 ? 0 : part * PS / DS, d1 = part < 0 ? 0 : (part + 1) * PS / DS;
    constexpr int NMF = TN * TM, NR = TN + TM;
#pragma unroll
    for (int idx = 0; idx < NMF; ++idx) {
      acc[idx / TM][idx % TM] = mfma32(wc[idx / TM], xc[idx % TM], acc[idx / TM][idx % TM]);
      if constexpr (rd && !W4) {
#pragma unroll
        for (int q = 0; q < NR; ++q)
          if ((q < NMF ? q : NMF - 1) == idx) {
            if (q == 0)
              read_w(rs, JN, 0, wn_);
            else if (q <= TM)
              read_x(rs, JN, q - 1, xn);
            else
              read_w(rs, JN, q - TM, wn_);
          }
      }
      if constexpr (rd && W4) {
        constexpr bool new_pair = (JN % 2) == 0;
        constexpr int NRD = TM + (new_pair ? TN : 0);
#pragma unroll
        for (int q = 0; q < NRD; ++q)
          if ((q < NMF ? q : NMF - 1) == idx) {
            if (q < TM)
              read_x(rs, JN, q, xn);
            else
              read_w(rs, JN, q - TM, raw);
          }
        // unpack of block a: in the last TN slots, and never before the slot
        // that reads its new chunk (TM + a, clamped; a slot issues its reads
        // before its unpacks).  At 64 x 128 (NMF = TN = 2) both land in slot 1.
#pragma unroll
        for (int a = 0; a < TN; ++a) {
          constexpr int first_slot = new_pair ? (NMF > TN ? NMF - TN : 0) : 0;
          const int want = first_slot + a > TM + a || !new_pair ? first_slot + a : TM + a;
          if ((want < NMF ? want : NMF - 1) == idx) unpack_half(a, JN % 2, wn_);
        }
      }
      if constexpr (part >= 0 && d1 > d0) {  // a part is empty when PS < DS
#pragma unroll
        for (int d = d0; d < d1; ++d)
          if ((d - d0) * NMF / (d1 - d0) == idx) dma_one(dst, dsl, d);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const int nk = (kloop > 0 ? kloop : K) / BK;  // k-stages (a split-K slice: kloop of K)
  i32x4 wf[2][TN], xf[2][TM];
  // Prologue: stages 0 .. NS-2 into slots 0 .. NS-2, and part 0 of stage
  // NS-1 into slot NS-1; stage 0's first sub-steps issue its other parts as
  // every stage does for the stage before, so the first stage needs no code
  // of its own (a copy of the loop body costs registers, and a spill reload
  // would wait for every DMA load in flight).  Every issue moves the same
  // loads per wave; a stage past the end reloads stage nk-1 into a slot that
  // is never read, so the loads in flight at each wait are always the same
  // count.
  constexpr int P0 = PS / DS;  // loads in part 0 of a stage
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int d = 0; d < (st < NS - 1 ? PS : P0); ++d) dma_one(min(st, nk - 1), st, d);
  wait_vmcnt<(NS - 2) * PS + P0>();  // stage 0 landed (loads complete in order)
  __syncthreads();
#pragma unroll
  for (int b = 0; b < TM; ++b) read_x(0, 0, b, xf[0]);
#pragma unroll
  for (int a = 0; a < TN; ++a) {
    if constexpr (W4) {
      read_w(0, 0, a, raw);
      unpack_half(a, 0, wf[0]);
    } else {
      read_w(0, 0, a, wf[0]);
    }
  }

  // Stage kt: sub-steps 0 .. SUBS-1.  The barrier before the last sub-step
  // publishes stage kt+1 (NS-2 younger stages still in flight) and frees the
  // slot of stage kt, which receives stage kt+NS from that sub-step on.  The
  // first DS-1 sub-steps issue the rest of the loads the previous stage began
  // (in the first stage, the rest of the prologue's stage NS-1).
  auto stage_body = [&](int kt, auto lastc) {
    constexpr bool LAST = decltype(lastc)::value != 0;
    const int sl = kt % NS;
    const int pdst = min(kt - 1 + NS, nk - 1), psl = (kt + NS - 1) % NS;
#define DMA_SUB(J)                                                                          \
  if constexpr ((J) < SUBS - 1) {                                                           \
    step(icst<(J) + 1>{}, icst<1>{}, icst<((J) + 1 < DS) ? (J) + 2 : 0>{},                   \
         wf[(J) & 1], xf[(J) & 1], sl, wf[((J) + 1) & 1], xf[((J) + 1) & 1], pdst, psl);     \
  } else if constexpr (!LAST) {                                                             \
    wait_vmcnt<(NS - 2) * PS>();                                                            \
    __syncthreads();                                                                        \
    step(icst<0>{}, icst<1>{}, icst<1>{}, wf[(J) & 1], xf[(J) & 1], (kt + 1) % NS, wf[0],   \
         xf[0], min(kt + NS, nk - 1), sl);                                                  \
  } else {                                                                                  \
    step(icst<0>{}, icst<0>{}, icst<0>{}, wf[(J) & 1], xf[(J) & 1], 0, wf[0], xf[0], 0, 0); \
  }
    DMA_SUB(0)
    DMA_SUB(1)
    if constexpr (SUBS == 4) {
      DMA_SUB(2)
      DMA_SUB(3)
    }
#undef DMA_SUB
  };
  for (int kt = 0; kt < nk - 1; ++kt) stage_body(kt, icst<0>{});
  // Last stage.  The per-channel epilogue's scales are requested here, so
  // their latency hides behind the last MFMAs; indices are clamped, so the
  // loads are unconditional.
  float sw_t = 0.0f, sa_t = 0.0f;
  uint16_t b_t = 0;
  if constexpr (EPI == EPI_PC) {
    sw_t = reinterpret_cast<const float*>(p.sw)[min(n0 + tid % BN, N - 1)];
    sa_t = p.sa[min(m0 + tid % BM, M - 1)];
    if (p.bias) b_t = p.bias[min(n0 + tid % BN, N - 1)];
  }
  stage_body(nk - 1, icst<1>{});
  wait_vmcnt<0>();  // the reloads past the end land before LDS is reused

  // ---- epilogue: lane holds, per 32x32 block and group g, 4 consecutive n
  //      n = nblk + 8g + 4 (lane / 32) + [0..3] of row m = mblk + lane % 32
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
    // LDS after the ring is released: [0, OUT) fp16 tile, then sw, sa, bias
    float* ssw = reinterpret_cast<float*>(smem + C::OUT);
    float* ssa = ssw + BN;
    uint16_t* sbias = reinterpret_cast<uint16_t*>(ssa + BM);
    __syncthreads();  // every wave is done with the ring
    if (tid < BN) {
      ssw[tid] = sw_t;
      sbias[tid] = b_t;
    }
    if (tid < BM) ssa[tid] = sa_t;
    __syncthreads();
    float sam[TM];
#pragma unroll
    for (int b = 0; b < TM; ++b) sam[b] = ssa[wm * WM + b * 32 + frow];
    // the bias test is uniform: taken once, outside the conversion loops (a
    // per-element select would cost two VALU ops per accumulator)
    // Every column scale this lane needs is read before the conversion, so no
    // LDS wait (which would also wait for the tile stores already issued)
    // sits inside it.
    f32x4 swv[TN][4];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        swv[a][g] = *reinterpret_cast<const f32x4*>(ssw + wn * WN + a * 32 + 8 * g + 4 * h);
    auto convert = [&](auto biasc) {
      constexpr bool BIAS = decltype(biasc)::value != 0;
      i32x2 bbv[TN][4];
      if constexpr (BIAS) {
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            bbv[a][g] = *reinterpret_cast<const i32x2*>(sbias + wn * WN + a * 32 + 8 * g + 4 * h);
      }
#pragma unroll
      for (int a = 0; a < TN; ++a) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int nl = wn * WN + a * 32 + 8 * g + 4 * h;  // column in tile
          float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          if constexpr (BIAS) {
            const i32x2 bb = bbv[a][g];
            bv[0] = h2f((uint16_t)((uint32_t)bb[0] & 0xffffu));
            bv[1] = h2f((uint16_t)((uint32_t)bb[0] >> 16));
            bv[2] = h2f((uint16_t)((uint32_t)bb[1] & 0xffffu));
            bv[3] = h2f((uint16_t)((uint32_t)bb[1] >> 16));
          }
#pragma unroll
          for (int b = 0; b < TM; ++b) {
            const int ml = wm * WM + b * 32 + frow;  // row in tile
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              // The volatile asm keeps each path's int -> float conversions
              // inside that path: hoisted above the bias test, the converted
              // accumulators were parked back in AGPRs and the 256 x 256 tile
              // spilled.
              int iv = acc[a][b][4 * g + r];
              asm volatile("" : "+v"(iv));
              float v = (float)iv * sam[b];
              v = v * swv[a][g][r];
              if constexpr (BIAS) v = v + bv[r];
              o[r] = v;
            }
            *reinterpret_cast<i32x2*>(smem + ml * C::OUT_LD + nl * 2) =
                i32x2{(int)f2h2(o[0], o[1]), (int)f2h2(o[2], o[3])};
          }
        }
      }
    };
    if (p.bias)
      convert(icst<1>{});
    else
      convert(icst<0>{});
    __syncthreads();
    // whole rows: BN / 8 lanes x 16 bytes per row, 512 / BN rows per store
    constexpr int LPR = BN / 8, RPS = 64 / LPR;
    const int cl = (lane % LPR) * 8;  // first column of this lane's 8
    const int n = n0 + cl;
#pragma unroll 4
    for (int rr = wave * RPS + lane / LPR; rr < BM; rr += NWV * RPS) {
      const int m = m0 + rr;
      if (m < M && n < N)
        *reinterpret_cast<i32x4*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + n) =
            *reinterpret_cast<const i32x4*>(smem + rr * C::OUT_LD + cl * 2);
    }
  }
}

// Uniform grid: one BM x BN tile per workgroup.
template <int BM, int BN, int BK, int EPI, int WF, int NWV = 4>
__global__ __launch_bounds__(64 * NWV, 1) void gemm_dma_kernel(const GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) int8_t smem[DmaCfg<BM, BN, BK, WF, NWV>::SMEM];
  int m0, n0;
  tile_coords<BM, BN>(xcd_remap(blockIdx.x, gridDim.x), p.M, 0, p.N, m0, n0);
  dma_tile<BM, BN, BK, EPI, WF, NWV>(p, m0, n0, smem);
}

// Two tile sizes in one grid, so that the last round of workgroups is not
// half empty: the big workgroups take 256 x 256 tiles of columns [0, nsplit),
// the small ones 128 x 256 tiles of columns [nsplit, N), twice as many tiles
// of half the work.  Workgroups start in index order: [0, s1) small tiles
// 0 .. s1-1, [s1, s1 + nbig) the big tiles, the rest the other small tiles.
// With s1 = half the small tiles, half the CUs start on a small tile and run
// half a tile out of phase with the other half from then on, so the tile
// epilogues' output stores (a 256 x 256 tile writes 128 KB, a round of
// tiles 32 MB at once, for about 4.6 us at M=4096 N=10240 K=2560) meet the
// other half's k-loops instead of each other (that shape: 102.0 -> 95.9 us,
// bit-identical).  Each region keeps its own XCD remap; s1 and nbig are
// multiples of 8, so a region's index keeps the XCD of its workgroup.
template <int EPI, int WF, int NWV = 4>
__global__ __launch_bounds__(64 * NWV, 1) void gemm_dma_mixed_kernel(const GemmArgs p, int nbig,
                                                                     int nsplit, int s1) {
  constexpr int S1 = DmaCfg<256, 256, 128, WF, NWV>::SMEM,
                S2 = DmaCfg<128, 256, 128, WF, NWV>::SMEM;
  __shared__ __attribute__((aligned(1024))) int8_t smem[S1 > S2 ? S1 : S2];
  const int b = blockIdx.x;
  int m0, n0;
  if (b >= s1 && b < s1 + nbig) {
    tile_coords<256, 256>(xcd_remap(b - s1, nbig), p.M, 0, nsplit, m0, n0);
    dma_tile<256, 256, 128, EPI, WF, NWV>(p, m0, n0, smem);
  } else {
    const int bs = b < s1 ? b : b - nbig;
    tile_coords<128, 256>(xcd_remap(bs, gridDim.x - nbig), p.M, nsplit, p.N, m0, n0);
    dma_tile<128, 256, 128, EPI, WF, NWV>(p, m0, n0, smem);
  }
}

namespace {

// 256-column tiles run eight waves (two per SIMD), the smaller tiles four.
template <int BM, int BN, int BK, int EPI, int WF = W_I8>
hipError_t run_dma(const GemmArgs& a, hipStream_t s) {
  constexpr int NWV = BN == 256 ? 8 : 4;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  gemm_dma_kernel<BM, BN, BK, EPI, WF, NWV><<<tiles, 64 * NWV, 0, s>>>(a);
  return hipGetLastError();
}

template <int EPI, int WF>
hipError_t pick_tile(const GemmArgs& a, hipStream_t s) {
  // Estimated time = rounds x tile area / tile rate.  Rates are throughputs
  // measured on MI355X relative to a 256 x 256 tile (= 1), with back-to-back
  // launches, over M = 128 .. 8192 and (N, K) from (10240, 2560) to
  // (4096, 12288).  A last round only partly full runs with less contention:
  // it counts 0.6 + 0.4 x its occupancy.  Ties go to the earlier candidate.
  // 192 x 256 (waves of 96 x 128) serves grids whose 256 x 256 tiles make one
  // partial round (int8: M=4096 N=2560 K=10240: 97.3 vs 105.8 us; M=1024
  // N=10240 K=2560: 33.5 vs 35.8 us; int4: M=1024 N=10240 K=2560: 38.6 vs
  // 42.8 us).  The mixed grid below reads candidates 0 and 1.
  struct Cand { int bm, bn; double rate; };
  static const Cand c8[] = {{256, 256, 1.0},   {128, 256, 0.87}, {128, 128, 0.75},
                            {128, 64, 0.517},  {64, 128, 0.508}, {64, 64, 0.40},
                            {192, 256, 0.90}};
  static const Cand c4[] = {{256, 256, 1.0},   {128, 256, 0.77}, {128, 128, 0.60},
                            {128, 64, 0.41},   {64, 128, 0.40},  {64, 64, 0.32},
                            {192, 256, 0.92}};
  const Cand* cands = WF == W_I4 ? c4 : c8;
  const int cus = num_cus();
  int best = 0;
  double best_cost = 1e300;
  for (int i = 0; i < 7; ++i) {
    const int64_t tiles =
        (int64_t)((a.M + cands[i].bm - 1) / cands[i].bm) * ((a.N + cands[i].bn - 1) / cands[i].bn);
    const int64_t full = tiles / cus, rest = tiles % cus;
    const double rounds = (double)full + (rest ? 0.6 + 0.4 * (double)rest / cus : 0.0);
    const double cost = rounds * cands[i].bm * cands[i].bn / cands[i].rate;
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = i;
    }
  }
  // Mixed grid: when the 256 x 256 tiles leave a last round at most half
  // full, made of whole tile columns, those columns can run as twice as many
  // 128 x 256 tiles of half the length, so the last round is full and half
  // as long.
  {
    const int tm = (a.M + 255) / 256, tn = (a.N + 255) / 256;
    const int64_t T = (int64_t)tm * tn;
    const int R = (int)(T % cus);
    if (T > cus && R > 0 && 2 * R <= cus && R % tm == 0) {
      const double tail = (0.6 + 0.4 * 2.0 * R / cus) * 128 * 256 / cands[1].rate;
      if ((double)(T / cus) * 256 * 256 / cands[0].rate + tail < best_cost * 0.999) {
        const int tail_cols = R / tm;
        const int nsplit = (tn - tail_cols) * 256;
        const int nbig = (int)(T - R);
        const int nsmall = ((a.M + 127) / 128) * tail_cols;
        // half the small tiles first (a multiple of 8), when the big region
        // starts on an XCD boundary; otherwise all of them last
        const int s1 = nbig % 8 == 0 ? nsmall / 2 / 8 * 8 : 0;
        gemm_dma_mixed_kernel<EPI, WF, 8><<<nbig + nsmall, 512, 0, s>>>(a, nbig, nsplit, s1);
        return hipGetLastError();
      }
    }
  }
  const int bm = cands[best].bm, bn = cands[best].bn;
  if (bm == 256) return run_dma<256, 256, 128, EPI, WF>(a, s);
  if (bm == 192) return run_dma<192, 256, 128, EPI, WF>(a, s);
  if (bm == 128 && bn == 256) return run_dma<128, 256, 128, EPI, WF>(a, s);
  if (bm == 128 && bn == 128) return run_dma<128, 128, 128, EPI, WF>(a, s);
  if (bm == 128) return run_dma<128, 64, 128, EPI, WF>(a, s);
  if (bn == 128) return run_dma<64, 128, 128, EPI, WF>(a, s);
  return run_dma<64, 64, 128, EPI, WF>(a, s);
}

}  // namespace

// Compute units of the current device (cached per device).
int num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// ---- Split-K for per-channel shapes whose tiles leave most CUs idle (M up
// to a few hundred rows on small N, e.g. M=128 N=2560 K=10240: 20 tiles of
// 128 x 128).  Workgroup (t, s) runs tile t over the k range [s ks, (s+1) ks)
// with the int32 epilogue into partial slice s; the dequant kernel sums the
// slices (int32: exact in any order) and applies the per-channel epilogue
// with the operation order of the tile epilogue, so the result is the same
// bits as one pass over K.
template <int BM>
__global__ __launch_bounds__(256, 1) void gemm_dma_splitk_kernel(const GemmArgs p, int ks,
                                                                 int32_t* __restrict__ part) {
  constexpr int BN = 128, BK = 128;
  __shared__ __attribute__((aligned(1024))) int8_t smem[DmaCfg<BM, BN, BK, W_I8>::SMEM];
  const int sl = blockIdx.y;
  GemmArgs q = p;
  q.x = p.x + (int64_t)sl * ks;
  q.w = reinterpret_cast<const int8_t*>(p.w) + (int64_t)sl * ks;
  q.y = part + (int64_t)sl * p.M * p.N;
  int m0, n0;
  tile_coords<BM, BN>(xcd_remap(blockIdx.x, gridDim.x), p.M, 0, p.N, m0, n0);
  dma_tile<BM, BN, BK, EPI_I32, W_I8>(q, m0, n0, smem, ks);
}

// y[m, n..n+3] = h(f32(f32(sum_s part[s][m][n]) * sa[m]) * sw[n] [+ bias[n]]);
// N % 4 == 0, so a thread's four columns share a row.
__global__ __launch_bounds__(256) void splitk_dequant_kernel(const GemmArgs p,
                                                             const int32_t* __restrict__ part,
                                                             int S) {
  const int64_t MN = (int64_t)p.M * p.N;
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= MN) return;
  const int m = (int)(e / p.N), n = (int)(e % p.N);
  i32x4 acc = *reinterpret_cast<const i32x4*>(part + e);
  for (int sl = 1; sl < S; ++sl) acc += *reinterpret_cast<const i32x4*>(part + sl * MN + e);
  const float sam = p.sa[m];
  const f32x4 swv = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.sw) + n);
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = (float)acc[r] * sam;
    v = v * swv[r];
    if (p.bias) v = v + h2f(p.bias[n + r]);
    o[r] = v;
  }
  *reinterpret_cast<i32x2*>(reinterpret_cast<uint16_t*>(p.y) + e) =
      i32x2{(int)f2h2(o[0], o[1]), (int)f2h2(o[2], o[3])};
}

// K slices for a per-channel int8 shape (1 = no split): only where the
// 128-column tiles (64-row for M <= 64) fill at most a quarter of the CUs,
// then the most slices, in powers of two, that keep the grid within one
// workgroup per CU and each slice at 8 k-stages or more.  Measured with the
// weights streaming from HBM (whole linears): N=2560 K=10240 M=32 / 128 /
// 256: 25.6 -> 17.9 us (8 slices), 32.3 -> 23.8 us (8), 32.6 -> 28.8 us (4);
// N=4096 K=12288 M=64: 37.1 -> 23.7 us (8).  Grids of more tiles gained
// little or lost (N=10240 K=2560 M=32, 80 tiles: 12.4 us whole, 16.2 us in
// two slices).  Nor where 64 x 64 tiles alone fill three quarters of the CUs
// (M=512 N=2048 K=2048: 18.1 us in two slices against 10.3-10.6 us unsplit on
// 256 tiles of 64 x 64; K=6144: 26.7-27.8 us in four against 21.5 us; whole
// linears, weights from HBM).  The caller also checks the alignment of the operands.  The
// tile's per-lane weight and activation offsets are 32-bit (up to 128 rows x
// K bytes, and the slices address the full row pitch K), so K * 256 must stay
// below 2^32 as for launch_gemm's DMA tiles.
int splitk_ways(int M, int N, int K) {
  if (M <= 16 || M > 512 || N % 8 != 0 || K % 128 != 0) return 1;
  if ((int64_t)K * 256 >= ((int64_t)1 << 32)) return 1;
  const int bm = M <= 64 ? 64 : 128;
  const int tiles = ((M + bm - 1) / bm) * ((N + 127) / 128);
  const int cus = num_cus();
  if (4 * tiles > cus) return 1;
  if ((int64_t)4 * ((M + 63) / 64) * ((N + 63) / 64) > (int64_t)3 * cus) return 1;
  int S = 1;
  while (S < 16 && tiles * 2 * S <= cus && K % (128 * 2 * S) == 0 && K / (2 * S) >= 1024) S *= 2;
  return S;
}

size_t splitk_bytes(int M, int N, int K) {
  const int S = splitk_ways(M, N, K);
  return S > 1 ? (size_t)S * M * N * 4 : 0;
}

hipError_t launch_gemm_splitk(const GemmArgs& a, int S, int32_t* part, hipStream_t s) {
  const int ks = a.K / S;
  if (a.M <= 64) {
    const dim3 grid(((a.M + 63) / 64) * ((a.N + 127) / 128), S);
    gemm_dma_splitk_kernel<64><<<grid, 256, 0, s>>>(a, ks, part);
  } else {
    const dim3 grid(((a.M + 127) / 128) * ((a.N + 127) / 128), S);
    gemm_dma_splitk_kernel<128><<<grid, 256, 0, s>>>(a, ks, part);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t quads = ((int64_t)a.M * a.N) / 4;
  splitk_dequant_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, s>>>(a, part, S);
  return hipGetLastError();
}

// Eligible: EPI_I32 or EPI_PC with int8 weights, EPI_PC with int4 weights;
// K % 128 == 0, N % 8 == 0, 16-byte aligned operands (launch_gemm checks).
hipError_t launch_gemm_dma(const GemmArgs& a, int epi, int wf, hipStream_t s) {
  if (wf == W_I4) return pick_tile<EPI_PC, W_I4>(a, s);
  if (epi == EPI_I32) return pick_tile<EPI_I32, W_I8>(a, s);
  return pick_tile<EPI_PC, W_I8>(a, s);
}

}  // namespace cider
