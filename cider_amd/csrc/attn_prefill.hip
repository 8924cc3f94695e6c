// Causal grouped-query attention of a prefill chunk over the KV cache.
//
//   for query i of the chunk (cache slot p = n - c + i), query head h of KV
//   head j = h / (H / KV):
//     s_t   = scale * q[i,h,:] . K[j,t,:]                 t <= p
//     o[i,h,:] = sum_t softmax(s)_t V[j,t,:]              -> fp16 [c, H, 128]
// with both caches [KV, T, 128] (position-major, as cider_qk_norm_rope writes
// them) and the chunk's own keys already in the cache (slots n - c .. n - 1).
// This is the attention the reference's prefill hands to MLX's fused SDPA
// (cider/fused_hybrid.py:179-196); MLX does not specify its accumulation
// order, so parity is within a tolerance of a float64 softmax attention.
//
// Numerics: scores are fp32 MFMA dot products of the fp16 operands; the
// softmax runs in base 2 with the scale folded into one fma per score
// (exp2(s * scale * log2 e - m)); probabilities are rounded to fp16 for the
// P.V MFMA (fp32 accumulation), and the row sum l is the MFMA sum of the same
// rounded probabilities, so numerator and denominator see one P.  The running
// max m is raised only when a block's max exceeds it by more than 8 (log2
// units): o and l share the reference, so the quotient is the same (up to
// rounding), p stays below 2^8 (well inside fp16), and the rescale of o runs
// for few blocks.  The output is o / l in fp32, rounded to fp16.
//
// MI355X design:
//   * a workgroup = 8 waves = one query head x 128 consecutive queries; wave
//     w holds queries 32 (w % 4) .. +31 of the block (its Q fragments live in
//     registers for the whole loop); the wave sets w / 4 = 0, 1 split the keys:
//     set s takes the 64-key blocks 2i + s.  The two sets' (m, l, o) are merged
//     through LDS at the end.  With 128 KB of LDS and 8 waves a workgroup
//     fills a CU (two waves per SIMD), and the hardware hands the next item to
//     whichever CU finishes first: items are ordered longest first (causal
//     blocks differ up to 16x in length), so the dispatch balances itself.
//   * scores: S^T = K Q^T with v_mfma_f32_32x32x16_f16 (K rows from LDS as
//     the A operand, Q as B), so each lane owns one query's column of scores:
//     the row max and exps are in-lane plus one exchange between the wave
//     halves.  P^T (fp16, straight from the score registers) is the B
//     operand of O^T += V^T P^T.
//   * K and V reach LDS by DMA (global_load_lds_dwordx4), double-buffered per
//     128-key stage, issued one stage ahead.  K rows keep 16-byte chunk c at
//     c ^ (row & 15) (the 16 lanes of a ds_read_b128 hit 16 bank groups);
//     V rows stay position-major and the V^T operand is read with gfx950's
//     transposing ds_read_b64_tr_b16 (lane i of each 16-lane group supplies
//     the address of 4 dims of one key; lane j receives dim j of 4 keys),
//     with chunk c of row r at c ^ 4 (r & 3) so its 64 lanes are conflict
//     free.  No register staging and no VALU for either operand.
//   * causal blocks: a wave skips blocks wholly past its queries and masks
//     only the blocks that cross its diagonal.
//   * with KV % 8 == 0 each XCD (workgroup i runs on XCD i % 8) serves the KV
//     heads j with j % 8 == its index, so its L2 holds only their K / V.
#include <type_traits>

#include "common.hpp"
#include "dma_common.hpp"
#include "kernels.hpp"
#include "quant_common.hpp"

namespace cider {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kD = 128;                    // head dimension
constexpr int kBKey = 64;                  // keys per wave block
constexpr int kBQ = 128;                   // queries per workgroup
constexpr int kThreads = 512;              // 8 waves
constexpr int kStage = 2 * kBKey;          // keys per stage (one block per wave set)
constexpr int kTile = kStage * kD * 2;     // one stage of K (or of V): 32 KB
constexpr int kK0 = 0, kV0 = 2 * kTile;    // K buffers at 0 / 32 KB, V buffers at 64 / 96 KB
constexpr int kSetBytes = kBKey * kD * 2;  // one wave set's block within a stage: 16 KB
constexpr float kRescaleLog2 = 8.0f;       // running-max slack (log2 units)

__device__ __forceinline__ f16x4 tr_load(const uint8_t* p) {
  typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fp16x4_t;
  auto lp = reinterpret_cast<__attribute__((address_space(3))) fp16x4_t*>(
      (__attribute__((address_space(3))) uint8_t*)p);
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(lp));
}

__device__ __forceinline__ f32x16 mfma_f16(i32x4 a, i32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// One workgroup = one item (query block qb, query head h) and one part of its
// keys: with P > 1 parts, part p takes stages [p * nst / P, (p + 1) * nst / P)
// of the item's nst stages and writes its unnormalised (o, m, l) to ws; the
// merge kernel combines the parts.  With P == 1 it writes the output.
__global__ __launch_bounds__(kThreads, 1) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, uint16_t* __restrict__ o, float* __restrict__ ws, int c,
    int n, const int64_t* __restrict__ n_dev, int H, int KV, int T, int P, float sc) {
  if (n_dev != nullptr) {  // the valid length from the device, within [c, the host bound]
    const int64_t nd = *n_dev;
    n = (int)(nd < c ? c : (nd > n ? n : nd));
  }
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * kTile];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;

  const int nqb = (c + kBQ - 1) / kBQ;
  int qb, h, part;
  if (KV % 8 == 0) {
    // XCD x = blockIdx.x % 8 takes KV heads j % 8 == x, longest items first.
    const int x = blockIdx.x & 7, s = blockIdx.x >> 3, per = H / 8, G = H / KV;
    qb = nqb - 1 - s / (per * P);
    const int r = (s / P) % per;
    part = s % P;
    h = ((r / G) * 8 + x) * G + r % G;
  } else {  // item i = blockIdx.x / P, longest first: query block nqb - 1 - i / H of head i % H
    const int i = (int)blockIdx.x / P;
    part = (int)blockIdx.x % P;
    qb = nqb - 1 - i / H;
    h = i % H;
  }
  const int j = h / (H / KV);
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qw = wave & 3, set = wave >> 2;
  const int wq0 = qb * kBQ + qw * 32;  // first query (chunk index) of the wave
  const int ql = wq0 + l32;            // this lane's query
  const int qabs = n - c + ql;         // its cache slot
  const int qa_lo = n - c + wq0;
  const int qa_hi = n - c + min(wq0 + 31, c - 1);
  const bool wave_live = wq0 < c;

  const int kend = n - c + min(qb * kBQ + kBQ, c);  // keys the item needs
  const int nst_item = (kend + kStage - 1) / kStage;
  const int st0 = part * nst_item / P, st1 = (part + 1) * nst_item / P;  // this part's stages
  const uint16_t* kbase = kc + (int64_t)j * T * kD;
  const uint16_t* vbase = vc + (int64_t)j * T * kD;

  i32x4 qf[8];  // Q fragments, loaded once the first stage's DMA is out

  // DMA: wave w fills rows 16w .. 16w + 15 of a stage, 4 rows per
  // instruction; the lane of LDS slot (row r, chunk p) fetches the global
  // chunk that the row's swizzle puts there.
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wave + 4 * i + (lane >> 4);
    koff[i] = (uint32_t)(r * (kD * 2) + 16 * ((lane & 15) ^ (r & 15)));
    voff[i] = (uint32_t)(r * (kD * 2) + 16 * ((lane & 15) ^ (4 * (r & 3))));
  }
  auto issue = [&](int st, int buf) {
    const int key0 = st * kStage;
    const uint32_t kl = lds0 + kK0 + buf * kTile + 16 * wave * (kD * 2);
    const uint32_t vl = lds0 + kV0 + buf * kTile + 16 * wave * (kD * 2);
    if (key0 + kStage <= n) {
      const uint16_t* kb = kbase + (int64_t)key0 * kD;
      const uint16_t* vb = vbase + (int64_t)key0 * kD;
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16s(kb, koff[i], kl + 4 * i * (kD * 2));
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16s(vb, voff[i], vl + 4 * i * (kD * 2));
    } else {  // the stage holding slot n - 1: rows past it repeat row n - 1 (masked; whatever
              // the cache holds there, even NaN, must not reach 0 * V in the P.V product)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * wave + 4 * i + (lane >> 4);
        const uint32_t row = (uint32_t)min(key0 + r, n - 1) * (kD * 2);
        dma16s(kbase, row + 16 * ((lane & 15) ^ (r & 15)), kl + 4 * i * (kD * 2));
        dma16s(vbase, row + 16 * ((lane & 15) ^ (4 * (r & 3))), vl + 4 * i * (kD * 2));
      }
    }
  };

  // K as the A operand: lane reads key 32kb + l32 of its set's block, dims
  // 16s + 8hl .. +7.
  uint32_t kaddr[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    kaddr[s] = (uint32_t)(kK0 + set * kSetBytes + l32 * (kD * 2) +
                          16 * ((2 * s + hl) ^ (l32 & 15)));
  // V^T as the A operand: lane l of 16-lane group G = l / 16 (i = l % 16,
  // e = i / 4, q = i % 4) points at key k0 + e, dims 32a + 16 (G & 1) + 4q;
  // the transposing read gives lane l dim 32a + 16 (G & 1) + i of keys
  // k0 .. k0 + 3, k0 = 32kb + 16mm + 4hl: the key order of the P^T registers.
  const int trG = lane >> 4, tre = (lane >> 2) & 3, trq = lane & 3;
  uint32_t vaddr[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int row = 4 * (trG >> 1) + tre;
    const int chunk = (4 * a + 2 * (trG & 1) + (trq >> 1)) ^ (4 * tre);
    vaddr[a] = (uint32_t)(kV0 + set * kSetBytes + row * (kD * 2) + 16 * chunk + 8 * (trq & 1));
  }

  f32x16 oacc[4], lacc;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[a][r] = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) lacc[r] = 0.0f;
  float m_i = -INFINITY;
  const i32x4 ones = {0x3C003C00, 0x3C003C00, 0x3C003C00, 0x3C003C00};  // fp16 1.0 x 8

  auto stage = [&](auto bufc, int st) {
    constexpr int buf = decltype(bufc)::value;  // compile-time: LDS offsets become immediates
    const bool more = st + 1 < st1;
    if (more) issue(st + 1, buf ^ 1);
    const int key0 = st * kStage + set * kBKey;  // this wave's block
    if (wave_live && key0 <= qa_hi) {
      // S^T = K Q^T: lane (query l32, half hl) gets keys 32kb + 8(r/4) + 4hl + r%4.
      f32x16 sacc[2];
      i32x4 kf[8][2];
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          kf[s][kb] = *reinterpret_cast<const i32x4*>(smem + kaddr[s] +
                                                       (buf * kTile + kb * 32 * (kD * 2)));
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) sacc[kb] = mfma_f16(kf[s][kb], qf[s], sacc[kb]);
      // LDS reads run two MFMAs ahead; the two score tiles alternate.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int s = 0; s < 6; ++s) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);

      if (key0 + kBKey - 1 > qa_lo) {  // the block crosses the wave's diagonal
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = key0 + kb * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
            if (key > qabs) sacc[kb][r] = -INFINITY;
          }
      }
      float mb = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mb = fmaxf(mb, sacc[kb][r]);
      mb = fmaxf(mb, __shfl_xor(mb, 32));
      if (__any(mb * sc > m_i * sc + kRescaleLog2)) {
        // A lane whose keys so far (in this wave set) are all masked keeps m = -inf; its o and
        // l are 0, and it must not form -inf - -inf.
        const float m_new = fmaxf(m_i, mb);
        const float alpha =
            m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f((m_i - m_new) * sc);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[a][r] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) lacc[r] *= alpha;
        m_i = m_new;
      }
      const float mc = m_i == -INFINITY ? 0.0f : m_i * sc;  // such a lane's p: exp2(-inf) = 0
      i32x4 pf[2][2];  // P^T as the B operand: 8 keys k0 + {0..3, 8..11} per (kb, mm)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          f16x8 ph;
#pragma unroll
          for (int t = 0; t < 8; ++t)
            ph[t] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][8 * mm + t], sc, -mc));
          pf[kb][mm] = __builtin_bit_cast(i32x4, ph);
        }
      // O^T += V^T P^T; the ones tile sums the same fp16 P into l.
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          const uint32_t k0off = (uint32_t)(buf * kTile + (kb * 32 + 16 * mm) * (kD * 2));
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            const f16x4 v0 = tr_load(smem + vaddr[a] + k0off);
            const f16x4 v1 = tr_load(smem + vaddr[a] + (k0off + 8 * (kD * 2)));
            const f16x8 av = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
            oacc[a] = mfma_f16(__builtin_bit_cast(i32x4, av), pf[kb][mm], oacc[a]);
          }
          lacc = mfma_f16(ones, pf[kb][mm], lacc);
        }
    }
    if (more) wait_vmcnt<0>();
    __syncthreads();
  };

  // The first stage's DMA goes out before the Q loads, so the two latencies overlap.
  if (st0 < st1) issue(st0, 0);
  // Q as the B operand: lane (query l32, half hl) holds dims 16s + 8hl .. +7.
  const int qlc = ql < c ? ql : c - 1;
#pragma unroll
  for (int s = 0; s < 8; ++s)
    qf[s] = *reinterpret_cast<const i32x4*>(q + ((int64_t)qlc * H + h) * kD + 16 * s + 8 * hl);
  // Use the Q registers here (the loads complete in order, after the DMA): the
  // compiler cannot see the DMA loads in its wait bookkeeping and would
  // otherwise wait for every load in flight before the first MFMA of each block.
#pragma unroll
  for (int s = 0; s < 8; ++s) asm volatile("" ::"v"(qf[s]));
  wait_vmcnt<0>();
  __syncthreads();
  for (int st = st0; st < st1; st += 2) {
    stage(std::integral_constant<int, 0>{}, st);
    if (st + 1 < st1) stage(std::integral_constant<int, 1>{}, st + 1);
  }
  const float l_i = lacc[0];  // every row of the ones tile holds the query's sum

  // merge: set 1 hands (m, l, o) to set 0 through LDS (free after the last barrier)
  float* mo = reinterpret_cast<float*>(smem);
  float* ml = mo + 4 * 64 * 64;
  if (set == 1) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r) mo[(qw * 64 + a * 16 + r) * 64 + lane] = oacc[a][r];
    ml[(qw * 2) * 64 + lane] = m_i;
    ml[(qw * 2 + 1) * 64 + lane] = l_i;
  }
  __syncthreads();
  if (set == 0 && ql < c && P > 1) {
    // partial of this part: o = o0 a0 + o1 a1 and l = l0 a0 + l1 a1 relative to m; a part in
    // which neither set saw a key of this query writes m = -inf, l = 0, o = 0.
    const float m1 = ml[(qw * 2) * 64 + lane], l1 = ml[(qw * 2 + 1) * 64 + lane];
    const float m = fmaxf(m_i, m1);
    const bool none = m == -INFINITY;
    const float a0 = none ? 0.0f : __builtin_amdgcn_exp2f((m_i - m) * sc);
    const float a1 = none ? 0.0f : __builtin_amdgcn_exp2f((m1 - m) * sc);
    const int64_t row = ((int64_t)part * c + ql) * H + h;
    float* wo = ws + row * kD;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = 4 * g + t;
          v[t] = oacc[a][r] * a0 + mo[(qw * 64 + a * 16 + r) * 64 + lane] * a1;
        }
        *reinterpret_cast<f32x4*>(wo + a * 32 + 8 * g + 4 * hl) = v;
      }
    if (hl == 0) {
      float* wml = ws + (int64_t)P * c * H * kD + row * 2;
      wml[0] = m;
      wml[1] = l_i * a0 + l1 * a1;
    }
  }
  if (set == 0 && ql < c && P == 1) {
    const float m1 = ml[(qw * 2) * 64 + lane], l1 = ml[(qw * 2 + 1) * 64 + lane];
    const float m = fmaxf(m_i, m1);  // finite: set 0 always sees key 0
    const float a0 = __builtin_amdgcn_exp2f((m_i - m) * sc);
    const float a1 = __builtin_amdgcn_exp2f((m1 - m) * sc);  // 0 when set 1 saw no key
    const float inv = 1.0f / (l_i * a0 + l1 * a1);
    const float s0 = a0 * inv, s1 = a1 * inv;
    uint16_t* orow = o + ((int64_t)ql * H + h) * kD;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = 4 * g + t;
          v[t] = (_Float16)(oacc[a][r] * s0 + mo[(qw * 64 + a * 16 + r) * 64 + lane] * s1);
        }
        *reinterpret_cast<f16x4*>(orow + a * 32 + 8 * g + 4 * hl) = v;
      }
  }
}

// Output dims d0 .. d0 + 7 of partial row `row` ((token, head) pair) merged
// over the P key parts in ws (P x rows x 128 fp32 numerators, then P x rows
// x (m, l)): each part weighted by exp2((m_p - max_p m) * sc), the sum
// divided by the weighted l, rounded to fp16 (8 halves, packed).
__device__ __forceinline__ i32x4 merge8(const float* __restrict__ ws, int64_t rows, int64_t row,
                                        int d0, int P, float sc) {
  const float* ml = ws + (int64_t)P * rows * kD;
  float M = -INFINITY;
  for (int p = 0; p < P; ++p) M = fmaxf(M, ml[((int64_t)p * rows + row) * 2]);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, L = 0.0f;
  for (int p = 0; p < P; ++p) {
    const int64_t pr = (int64_t)p * rows + row;
    const float mp = ml[pr * 2];
    const float w = mp == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((mp - M) * sc);
    L += ml[pr * 2 + 1] * w;
    const f32x4 a = *reinterpret_cast<const f32x4*>(ws + pr * kD + d0);
    const f32x4 b = *reinterpret_cast<const f32x4*>(ws + pr * kD + d0 + 4);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc[t] += a[t] * w;
      acc[4 + t] += b[t] * w;
    }
  }
  const float inv = 1.0f / L;
  i32x4 v;
#pragma unroll
  for (int t = 0; t < 4; ++t) v[t] = (int32_t)f2h2(acc[2 * t] * inv, acc[2 * t + 1] * inv);
  return v;
}

// out[i, h, :] = sum_p o_p 2^((m_p - M) sc) / sum_p l_p 2^((m_p - M) sc), M = max_p m_p:
// 16 threads per (query, head), 8 dimensions each, parts in order.
__global__ __launch_bounds__(256) void attn_prefill_merge_kernel(const float* __restrict__ ws,
                                                                 uint16_t* __restrict__ out,
                                                                 int64_t rows, int P, float sc) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int d0 = 8 * (threadIdx.x & 15);
  if (row >= rows) return;
  *reinterpret_cast<i32x4*>(out + row * kD + d0) = merge8(ws, rows, row, d0, P, sc);
}

// The merge with the per-token quantization of the o projection's input
// fused in (cider/kernels/w8a8_quantize.metal:33-86, the helpers of
// quantize_per_token): one workgroup per token, its H heads x 128 dims as
// H * 16 vectors of 8, NVB per thread.  The fp16 values are those the merge
// kernel stores, so q and sa are bit-identical to that kernel followed by
// quantize_per_token, without the fp16 round trip through HBM.
template <int NVB>
__global__ __launch_bounds__(256) void attn_prefill_merge_quant_kernel(
    const float* __restrict__ ws, int8_t* __restrict__ qo, float* __restrict__ sa, int H,
    int64_t rows, int P, float sc) {
  __shared__ float red[4];
  const int64_t tok = blockIdx.x;
  const int nvec = H * (kD / 8);
  i32x4 v[NVB];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int e = threadIdx.x + 256 * i;
    if (e < nvec) {
      v[i] = merge8(ws, rows, tok * H + (e >> 4), 8 * (e & 15), P, sc);
      amax = absmax8(v[i], amax);
    }
  }
  amax = block_max4(amax, red);
  const float s = row_scale(amax);
  const float inv = 1.0f / s;
  if (threadIdx.x == 0) sa[tok] = s;
  int8_t* qr = qo + tok * H * kD;
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int e = threadIdx.x + 256 * i;
    if (e < nvec) *reinterpret_cast<i32x2*>(qr + 8 * e) = quant8(v[i], inv);
  }
}

}  // namespace

int attn_prefill_parts(int c, int n, int H) {
  const int items = ((c + kBQ - 1) / kBQ) * H;
  const int cus = num_cus();
  if (items >= cus) return 1;
  const int nst_max = (n + kStage - 1) / kStage;  // the longest item's stages
  int P = cus / items;
  P = P < 8 ? P : 8;
  P = P < nst_max / 4 ? P : nst_max / 4;  // at least four stages per part
  return P > 1 ? P : 1;
}

size_t attn_prefill_ws_floats(int c, int n, int H) {
  const int P = attn_prefill_parts(c, n, H);
  return P > 1 ? (size_t)P * c * H * (kD + 2) : 0;
}

hipError_t launch_attn_prefill(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                               uint16_t* out, float scale, float* ws, size_t ws_floats, int c,
                               int n, const int64_t* n_dev, int H, int KV, int64_t T,
                               hipStream_t s) {
  const float sc = scale * 1.4426950408889634f;
  int P = attn_prefill_parts(c, n, H);
  if (ws == nullptr || ws_floats < (size_t)P * c * H * (kD + 2)) P = 1;
  const int items = ((c + kBQ - 1) / kBQ) * H;
  attn_prefill_kernel<<<items * P, kThreads, 0, s>>>(q, kc, vc, out, ws, c, n, n_dev, H, KV,
                                                      (int)T, P, sc);
  if (P > 1) {
    const int64_t rows = (int64_t)c * H;
    attn_prefill_merge_kernel<<<(unsigned)((rows + 15) / 16), 256, 0, s>>>(ws, out, rows, P, sc);
  }
  return hipGetLastError();
}

size_t attn_prefill_quant_ws_bytes(int c, int n, int H) {
  const size_t f = attn_prefill_ws_floats(c, n, H) * sizeof(float);
  const size_t h = (size_t)c * H * kD * sizeof(uint16_t);
  return f > h ? f : h;
}

hipError_t launch_attn_prefill_quant(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                                     int8_t* qo, float* sa, float scale, void* ws,
                                     size_t ws_bytes, int c, int n, const int64_t* n_dev, int H,
                                     int KV, int64_t T, hipStream_t s) {
  const int P = attn_prefill_parts(c, n, H);
  const size_t part_bytes = (size_t)P * c * H * (kD + 2) * sizeof(float);
  if (P == 1 || ws_bytes < part_bytes) {
    // one part: the fp16 output in the workspace, then the row quantization
    uint16_t* out = reinterpret_cast<uint16_t*>(ws);
    hipError_t e = launch_attn_prefill(q, kc, vc, out, scale, nullptr, 0, c, n, n_dev, H, KV, T, s);
    if (e != hipSuccess) return e;
    return launch_quantize(out, qo, sa, c, H * kD, s);
  }
  const float sc = scale * 1.4426950408889634f;
  const int items = ((c + kBQ - 1) / kBQ) * H;
  float* wf = reinterpret_cast<float*>(ws);
  attn_prefill_kernel<<<items * P, kThreads, 0, s>>>(q, kc, vc, nullptr, wf, c, n, n_dev, H, KV,
                                                      (int)T, P, sc);
  const int64_t rows = (int64_t)c * H;
  const int nvec = H * (kD / 8);
  if (nvec <= 256)
    attn_prefill_merge_quant_kernel<1><<<c, 256, 0, s>>>(wf, qo, sa, H, rows, P, sc);
  else if (nvec <= 512)
    attn_prefill_merge_quant_kernel<2><<<c, 256, 0, s>>>(wf, qo, sa, H, rows, P, sc);
  else if (nvec <= 1024)
    attn_prefill_merge_quant_kernel<4><<<c, 256, 0, s>>>(wf, qo, sa, H, rows, P, sc);
  else
    attn_prefill_merge_quant_kernel<8><<<c, 256, 0, s>>>(wf, qo, sa, H, rows, P, sc);
  return hipGetLastError();
}

}  // namespace cider
