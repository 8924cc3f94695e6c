// Small-M int8 GEMM (M <= 16; int8 or packed int4 weights; per-channel,
// int32 or per-group epilogue) as a weight stream through LDS.
//
// Semantics are those of the other GEMM kernels, bit for bit:
//   EPI_I32 cider/kernels/w8a8_matmul.metal:301-453
//   EPI_PC  cider/kernels/w8a8_matmul.metal:63-81 (int8 weights, with bias);
//           cider/kernels/w4a8_matmul.metal:47-89 (int4 weights, no bias)
//   EPI_PG  cider/kernels/pergroup_int8_gemm.metal:152-189: one sequential
//           fp32 chain per output over the groups in order
//
// MI355X layout
//   * A workgroup of 4 waves owns RB blocks of 16 weight rows (n0 ..
//     n0 + 16 RB - 1) and every activation row (M <= MB, MB = 8 or 16).  K
//     arrives in stages of 512: the stage's weight rows (512 B, or 256 B of
//     packed int4), activation rows (512 B) and, per-group, the group scales
//     of the block's columns go global -> LDS by global_load_lds_dwordx4 into
//     a ring of NS stages.  A 1 KB instruction covers whole row pieces (two
//     or four rows of one stage); an MFMA operand load straight from HBM
//     touches 16 rows x 64 B per instruction and moves fewer bytes per cycle.
//     Each wave issues a fixed number of loads per stage, so a stage is
//     waited for by a constant vmcnt.
//   * LDS slot of 16-byte chunk c of row r: r * (row bytes) + 16 * (c ^ (r %
//     16)).  The DMA lane that writes a slot fetches the chunk that belongs
//     there, so the 16 rows one operand read touches at a k-slice fall in 16
//     distinct 16-byte bank groups.
//   * Wave w takes k-steps 2w and 2w + 1 (64 k each) of every stage: lane
//     (r = l % 16, q = l / 16) holds k in [64 t + 16 q, +16) of its row
//     (8 packed bytes for int4, unpacked in registers), and
//     v_mfma_i32_16x16x64_i8 takes the weights as A and the activations as B.
//   * Per-channel / int32: the int32 tiles accumulate over all stages, then
//     the four waves' tiles are summed through LDS (exact in any order) and
//     wave rb runs the epilogue of block rb.
//   * Per-group: a stage holds 8, 4 or 2 groups (gs 64, 128, 256).  Each wave
//     writes its int32 group sums of the stage (per k-step at gs 64, per wave
//     at gs 128, and half a group at gs 256) to LDS; after a barrier the owner
//     of each output adds the halves (int32, exact), and chains
//     acc = acc + f32(f32(D_g) * sw[g, n]) over the stage's groups in order.
//     The owners are eight more waves that only chain: while the MFMA waves
//     compute stage st into one parts buffer (and copy its scale block
//     beside it), the chain waves add up stage st - 1 from the other, so the
//     chain (1-4.4 us per call when the MFMA waves ran it between stages)
//     overlaps the stream; one barrier per stage orders both buffers.
#include "common.hpp"
#include "dma_common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

constexpr int kSdBK = 512;  // k per stage
constexpr int kSdKW = 4;    // MFMA waves per workgroup (two 64-wide k-steps each per stage)
constexpr int kSdCW = 8;    // per-group: chain waves beside them

template <int RB, int MB, int NS, int WF, int EPI, int GS, bool SWH>
struct SdCfg {
  static constexpr bool PG = EPI == EPI_PG;
  static constexpr int ROWS = 16 * RB;
  static constexpr int WB = WF == W_I4 ? kSdBK / 2 : kSdBK;  // weight bytes per row and stage
  static constexpr int CPRW = WB / 16, CPRX = kSdBK / 16;      // 16-byte chunks per row
  static constexpr int WS = ROWS * WB, XS = MB * kSdBK;
  static constexpr int ESZ = SWH ? 2 : 4;                      // group scale bytes
  static constexpr int GPS = PG ? kSdBK / GS : 0;              // groups per stage
  static constexpr int SROW = ROWS * ESZ;                      // scale bytes of a group row
  static constexpr int NSI = (GPS * SROW + 1023) / 1024;       // scale instructions per stage
  static constexpr int STAGE = WS + XS + NSI * 1024;
  static constexpr int NWI = WS / 1024, NXI = XS / 1024;
  static constexpr int PW = (NWI + NXI) / kSdKW;               // per wave and stage (+1: scales)
  static constexpr int RING = NS * STAGE;
  static constexpr int PARTS = PG ? (GS == 64 ? 8 : 4) : 0;    // int32 sums per stage
  static constexpr int TERMS = PARTS * ROWS * 16 * 4;
  // per-group: two buffers of a stage's parts and of its scale block
  static constexpr int CHAIN = PG ? 2 * (TERMS + NSI * 1024) : 0;
  static constexpr int RED = kSdKW * RB * 64 * 16;             // partial tiles (PC / I32)
  static constexpr int SMEM = (RING + CHAIN) > RED ? (RING + CHAIN) : RED;
  static_assert(NWI % kSdKW == 0 && NXI % kSdKW == 0, "whole DMA instructions per wave");
  static_assert(CPRW >= 16 && NSI <= kSdKW, "swizzle range; one scale instruction per wave");
  static_assert(RB <= kSdKW, "one wave per block in the epilogue");
  static_assert(NS >= 2 && (NS - 2) * (PW + 1) <= 63, "vmcnt range");
  static_assert(SMEM <= kLdsBytes, "LDS budget");
};

// Waits for the oldest outstanding stage of this wave when `rem` (0 ..
// NS - 2) later stages have been issued after it, P loads per stage.
template <int P, int NS, int R = NS - 2>
__device__ __forceinline__ void wait_stage(int rem) {
  if constexpr (R == 0) {
    wait_vmcnt<0>();
  } else {
    if (rem >= R) {
      wait_vmcnt<P * R>();
      return;
    }
    wait_stage<P, NS, R - 1>(rem);
  }
}

}  // namespace

template <int RB, int MB, int NS, int WF, int EPI, int GS, bool SWH>
__global__ __launch_bounds__((EPI == EPI_PG ? kSdKW + kSdCW : kSdKW) * 64) void skinny_dma_kernel(
    const GemmArgs p) {
  using C = SdCfg<RB, MB, NS, WF, EPI, GS, SWH>;
  constexpr bool PG = C::PG;
  constexpr int PW = C::PW, CPRW = C::CPRW, CPRX = C::CPRX, WB = C::WB;
  __shared__ __attribute__((aligned(1024))) int8_t smem[C::SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int n0 = blockIdx.x * C::ROWS;
  const int nst = K / kSdBK;
  const int64_t ldw = WF == W_I4 ? K / 2 : K;
  const int8_t* wbase = reinterpret_cast<const int8_t*>(p.w) + (int64_t)n0 * ldw;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  // Per-lane source offsets of this wave's PW instructions of a stage
  // (stage-invariant; a stage advances the scalar bases).  Instruction
  // i = wave + 4 j of the stage: the first NWI carry weight rows, the rest
  // activation rows, so j < NWI / 4 decides which at compile time.
  constexpr int JW = C::NWI / kSdKW;
  uint32_t off[PW];
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int i = wave + kSdKW * j;
    if (j < JW) {
      const int s = i * 64 + lane, r = s / CPRW, c = (s % CPRW) ^ (r & 15);
      off[j] = (uint32_t)(min(n0 + r, N - 1) - n0) * (uint32_t)ldw + 16u * (uint32_t)c;
    } else {
      const int s = (i - C::NWI) * 64 + lane, r = s / CPRX, c = (s % CPRX) ^ (r & 15);
      off[j] = (uint32_t)min(r, M - 1) * (uint32_t)K + 16u * (uint32_t)c;
    }
  }
  // per-group: wave w < NSI also loads chunk (64 w + lane) of the stage's
  // scale block [group][column n0 ..], columns past N from the row's last
  // valid chunk, lanes past the block from its first
  uint32_t soff = 0;
  if constexpr (PG) {
    const int b = (wave * 64 + lane) * 16;
    const int g = b / C::SROW;
    const int last = (N - n0) * C::ESZ / 16 - 1;  // N % 8 == 0: whole chunks
    soff = g < C::GPS ? (uint32_t)g * (uint32_t)N * C::ESZ + 16u * min((b % C::SROW) / 16, last) : 0u;
  }
  const bool sdma = PG && wave < C::NSI;
  auto issue = [&](int st) {
    const uint32_t slot = lds0 + (uint32_t)((st % NS) * C::STAGE);
    const int8_t* wsrc = wbase + (int64_t)st * WB;
    const int8_t* xsrc = p.x + (int64_t)st * kSdBK;
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      const int i = wave + kSdKW * j;
      if (j < JW)
        dma16s_nt(wsrc, off[j], __builtin_amdgcn_readfirstlane(slot + i * 1024));
      else
        dma16s(xsrc, off[j], __builtin_amdgcn_readfirstlane(slot + C::WS + (i - C::NWI) * 1024));
    }
    if constexpr (PG) {
      if (sdma) {
        const int8_t* ssrc = reinterpret_cast<const int8_t*>(p.sw) +
                             ((int64_t)st * C::GPS * N + n0) * C::ESZ;
        dma16s(ssrc, soff, __builtin_amdgcn_readfirstlane(slot + C::WS + C::XS + wave * 1024));
      }
    }
  };
  auto wait = [&](int rem) {
    if (sdma)
      wait_stage<PW + 1, NS>(rem);
    else
      wait_stage<PW, NS>(rem);
  };

  // MFMA operands of k-step t (0..7) of a stage slot
  const int xr = lr & (MB - 1);  // lanes past MB re-read rows: columns past M are not stored
  auto operand_w = [&](const int8_t* slot, int rb, int t) -> i32x4 {
    const int8_t* row = slot + (16 * rb + lr) * WB;
    if constexpr (WF == W_I4) {
      // 8 packed bytes: k in [64 t + 16 q, +16) is byte 32 t + 8 q of the row
      const int c = 2 * t + (lq >> 1);
      const i32x2 v = *reinterpret_cast<const i32x2*>(row + 16 * (c ^ lr) + 8 * (lq & 1));
      uint32_t e0, e1, e2, e3;
      unpack_w4_word((uint32_t)v[0], e0, e1);
      unpack_w4_word((uint32_t)v[1], e2, e3);
      return i32x4{(int)e0, (int)e1, (int)e2, (int)e3};
    } else {
      return *reinterpret_cast<const i32x4*>(row + 16 * ((4 * t + lq) ^ lr));
    }
  };
  auto operand_x = [&](const int8_t* slot, int t) -> i32x4 {
    return *reinterpret_cast<const i32x4*>(slot + C::WS + xr * kSdBK + 16 * ((4 * t + lq) ^ xr));
  };

  // per-group workgroups have eight more waves, which only run the chain
  const bool mma = wave < kSdKW;

  // The per-channel epilogue's operands, requested before the first weight
  // load so that their latency overlaps the stream instead of following it
  // (clamped: operands of outputs past N or M are loaded but not used).  Wave
  // rb < RB stores block rb, lane (r, q) columns n0 + 16 rb + 4 q .. + 3 of
  // row r.  (Measured: per-channel M=16 N=10240 K=2560 9.34 -> 9.02 us; the
  // per-group chain waves ran 3 % slower with their operands requested early.)
  float e_sa = 0.0f;
  f32x4 e_sw = {0.0f, 0.0f, 0.0f, 0.0f};
  uint16_t e_b[4] = {0, 0, 0, 0};
  if constexpr (EPI == EPI_PC) {
    if (wave < RB) {
      const int ncol = min(n0 + 16 * wave + 4 * lq, N - 4);
      e_sa = p.sa[min(lr, M - 1)];
      e_sw = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p.sw) + ncol);
#pragma unroll
      for (int r = 0; r < 4; ++r) e_b[r] = p.bias ? p.bias[ncol + r] : (uint16_t)0;
    }
  }
#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (mma && st < nst) issue(st);

  if constexpr (!PG) {
    i32x4 acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = i32x4{0, 0, 0, 0};
    for (int st = 0; st < nst; ++st) {
      wait(min(NS - 2, nst - 1 - st));
      __syncthreads();  // every wave's loads of stage st have landed; slot st-1 is free
      if (st + NS - 1 < nst) issue(st + NS - 1);
      const int8_t* slot = smem + (st % NS) * C::STAGE;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = 2 * wave + j;
        const i32x4 b = operand_x(slot, t);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma_i8(operand_w(slot, rb, t), b, acc[rb]);
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
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[r] = (float)v4[r] * e_sa;
        v[r] = v[r] * e_sw[r];
        if (p.bias) v[r] = v[r] + h2f(e_b[r]);
      }
      *reinterpret_cast<i32x2*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * N + ncol) =
          i32x2{(int)f2h2(v[0], v[1]), (int)f2h2(v[2], v[3])};
    }
  } else {
    // ---- per-group.  Parts of a stage (int32 sums in LDS, [part][output],
    // output o = (rb * 64 + lane) * 4 + r, the MFMA's C layout):
    //   gs 64: part 2 w + j = k-step 2 w + j = group 2 w + j
    //   gs 128: part w = group w;  gs 256: parts 2 g and 2 g + 1 = group g
    constexpr int NOUT = C::ROWS * 16;
    constexpr int NCH = kSdCW * 64;                 // chain threads (waves 4 .. 11)
    constexpr int OWN = (NOUT + NCH - 1) / NCH;     // outputs per chain thread (RB)
    constexpr int SB = C::NSI * 1024;               // scale block bytes
    auto parts = [&](int b) { return reinterpret_cast<int32_t*>(smem + C::RING + b * C::TERMS); };
    auto sbuf = [&](int b) { return smem + C::RING + 2 * C::TERMS + b * SB; };
    const int ct = tid - kSdKW * 64;                // chain thread index (chain waves)
    float facc[OWN];
#pragma unroll
    for (int o = 0; o < OWN; ++o) facc[o] = 0.0f;
    // chain of one stage: output idx adds the stage's groups in order
    auto chain = [&](const int32_t* pt, const int8_t* sc) {
#pragma unroll
      for (int o = 0; o < OWN; ++o) {
        const int idx = ct + o * NCH;
        if (NOUT % NCH != 0 && idx >= NOUT) continue;
        const int l = (idx >> 2) & 63;
        const int nl = 16 * (idx >> 8) + 4 * (l >> 4) + (idx & 3);  // column - n0
#pragma unroll
        for (int g = 0; g < C::GPS; ++g) {
          int32_t dg;
          if constexpr (GS == 256)
            dg = pt[(2 * g) * NOUT + idx] + pt[(2 * g + 1) * NOUT + idx];
          else
            dg = pt[g * NOUT + idx];
          float s;
          if constexpr (SWH)
            s = h2f(reinterpret_cast<const uint16_t*>(sc)[g * C::ROWS + nl]);
          else
            s = reinterpret_cast<const float*>(sc)[g * C::ROWS + nl];
          facc[o] = facc[o] + (float)dg * s;
        }
      }
    };
    for (int st = 0; st < nst; ++st) {
      if (mma) wait(min(NS - 2, nst - 1 - st));
      // stage st landed; slot st-1 is free; the parts and scales of stage st-1
      // are written, and the chain of stage st-2 has read its buffers
      __syncthreads();
      if (mma) {
        if (st + NS - 1 < nst) issue(st + NS - 1);
        const int8_t* slot = smem + (st % NS) * C::STAGE;
        int32_t* pt = parts(st & 1);
        i32x4 d[2][RB];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int t = 2 * wave + j;
          const i32x4 b = operand_x(slot, t);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            d[j][rb] = mfma_i8(operand_w(slot, rb, t), b,
                               (GS == 64 || j == 0) ? i32x4{0, 0, 0, 0} : d[0][rb]);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          if constexpr (GS == 64) {
            *reinterpret_cast<i32x4*>(pt + ((2 * wave) * NOUT) + (rb * 64 + lane) * 4) = d[0][rb];
            *reinterpret_cast<i32x4*>(pt + ((2 * wave + 1) * NOUT) + (rb * 64 + lane) * 4) =
                d[1][rb];
          } else {
            *reinterpret_cast<i32x4*>(pt + (wave * NOUT) + (rb * 64 + lane) * 4) = d[1][rb];
          }
        }
        // the scale block of the stage, for the chain of the next iteration
        // (the slot is reloaded before then); wave w copied-in kilobyte w
        if (sdma)
          *reinterpret_cast<i32x4*>(sbuf(st & 1) + wave * 1024 + lane * 16) =
              *reinterpret_cast<const i32x4*>(slot + C::WS + C::XS + wave * 1024 + lane * 16);
      } else if (st > 0) {
        chain(parts((st - 1) & 1), sbuf((st - 1) & 1));
      }
    }
    __syncthreads();
    if (mma) return;
    chain(parts((nst - 1) & 1), sbuf((nst - 1) & 1));
    // output idx = (rb, lane, r): weight row n0 + 16 rb + 4 (lane / 16) + r,
    // activation row lane % 16
#pragma unroll
    for (int o = 0; o < OWN; ++o) {
      const int idx = ct + o * NCH;
      if (NOUT % NCH != 0 && idx >= NOUT) continue;
      const int l = (idx >> 2) & 63;
      const int n = n0 + 16 * (idx >> 8) + 4 * (l >> 4) + (idx & 3), m = l & 15;
      if (m >= M || n >= N) continue;
      float v = facc[o] * p.sa[m];
      if (p.bias) v = v + h2f(p.bias[n]);
      reinterpret_cast<uint16_t*>(p.y)[(int64_t)m * N + n] = f2h(v);
    }
  }
}

namespace {

template <int RB, int MB, int WF, int EPI, int GS, bool SWH, int NS>
hipError_t run_sd_ns(const GemmArgs& a, hipStream_t s) {
  const int rows = 16 * RB;
  skinny_dma_kernel<RB, MB, NS, WF, EPI, GS, SWH>
      <<<(a.N + rows - 1) / rows, (EPI == EPI_PG ? kSdKW + kSdCW : kSdKW) * 64, 0, s>>>(a);
  return hipGetLastError();
}

// Ring slots: 4, or as many as the LDS holds beside the per-group buffers.
// Deeper rings measured slower (int4 gs 128 M=16 N=12288 K=4096: 7 slots
// 15.2 us against 13.9 us with 4; N=2560 K=10240 gs 128: 8 slots 15.3 us
// against 13.8 us).
template <int RB, int MB, int WF, int EPI, int GS, bool SWH>
constexpr int sd_slots() {
  using C2 = SdCfg<RB, MB, 2, WF, EPI, GS, SWH>;
  const int ns = (kLdsBytes - C2::CHAIN) / C2::STAGE;
  return ns > 4 ? 4 : ns;
}

template <int RB, int MB, int WF, int EPI, int GS, bool SWH>
hipError_t run_sd(const GemmArgs& a, hipStream_t s) {
  constexpr int NS = sd_slots<RB, MB, WF, EPI, GS, SWH>();
  return run_sd_ns<RB, MB, WF, EPI, GS, SWH, NS>(a, s);
}

// The fewest blocks of 16 rows per workgroup whose grid fills at most one
// workgroup per CU (every workgroup reads all activation rows, so fewer,
// taller workgroups read them fewer times); 4 past three blocks per CU.
template <int MB, int WF, int EPI, int GS, bool SWH>
hipError_t pick_rb_sd(const GemmArgs& a, hipStream_t s) {
  const int cus = num_cus();
  const int blocks = (a.N + 15) / 16;
  if (blocks <= cus) return run_sd<1, MB, WF, EPI, GS, SWH>(a, s);
  if (blocks <= 2 * cus) return run_sd<2, MB, WF, EPI, GS, SWH>(a, s);
  if (blocks <= 3 * cus) return run_sd<3, MB, WF, EPI, GS, SWH>(a, s);
  return run_sd<4, MB, WF, EPI, GS, SWH>(a, s);
}

template <int WF, int EPI, int GS, bool SWH>
hipError_t pick_mb_sd(const GemmArgs& a, hipStream_t s) {
  if (a.M <= 8) return pick_rb_sd<8, WF, EPI, GS, SWH>(a, s);
  return pick_rb_sd<16, WF, EPI, GS, SWH>(a, s);
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// Shapes the kernel takes: 1 <= M <= 16, K % 512 == 0 with at least 3 stages
// (K >= 1536), K * 64 < 2^32, N % 4 == 0 (N % 8 == 0 per-group), per-group
// gs 64 / 128 / 256 with fp32 scales (int4 weights: 64 / 128 with fp16
// scales), 16-byte aligned operands.
bool skinny_dma_supported(const GemmArgs& a, int wf, int epi, bool sw_half, int gs) {
  if (a.M < 1 || a.M > 16 || a.K % kSdBK != 0 || a.K / kSdBK < 3 || a.N % 4 != 0) return false;
  if ((int64_t)a.K * 64 >= ((int64_t)1 << 32)) return false;
  if (!al16(a.x) || !al16(a.w) || !al16(a.y)) return false;
  if (epi != EPI_I32 && !al16(a.sw)) return false;
  if (epi == EPI_I32 && wf != W_I8) return false;
  if (epi == EPI_PG) {
    if (a.N % 8 != 0 || sw_half != (wf == W_I4)) return false;
    if (gs != 64 && gs != 128 && !(gs == 256 && wf == W_I8)) return false;
  }
  return true;
}

hipError_t launch_skinny_dma(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s) {
  if (epi == EPI_I32) return pick_mb_sd<W_I8, EPI_I32, 0, false>(a, s);
  if (epi == EPI_PC) {
    if (wf == W_I4) return pick_mb_sd<W_I4, EPI_PC, 0, false>(a, s);
    return pick_mb_sd<W_I8, EPI_PC, 0, false>(a, s);
  }
  if (wf == W_I4) {
    // int4 weights come with fp16 group scales
    if (gs == 64) return pick_mb_sd<W_I4, EPI_PG, 64, true>(a, s);
    return pick_mb_sd<W_I4, EPI_PG, 128, true>(a, s);
  }
  if (gs == 64) return pick_mb_sd<W_I8, EPI_PG, 64, false>(a, s);
  if (gs == 128) return pick_mb_sd<W_I8, EPI_PG, 128, false>(a, s);
  return pick_mb_sd<W_I8, EPI_PG, 256, false>(a, s);
}

}  // namespace cider
