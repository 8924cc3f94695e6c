// Producer kernels of the W8A8 linear: the ops that hand a linear its input,
// with the per-token quantization of cider/kernels/w8a8_quantize.metal:33-86
// fused into their last pass, so the fp16 activation never makes a round trip
// through HBM before the GEMM reads its int8 copy.
//
//   rmsnorm_quant   h = x (+ add, rounded to fp16 and written back)
//                   r = 1 / sqrt(sum_k h^2 / K + eps)          (fp32)
//                   y = h(f32(w) * f32(h(h * r)))              (fp16 out, optional)
//                   q, sa = quantize_per_token(y)              (optional)
//                   The RMSNorm order is the Hugging Face / mlx-lm one that the
//                   reference's models use before every linear: normalise in
//                   fp32, round to fp16, then scale by the fp16 weight.
//   silu_mul_quant  y = h(f32(h(silu(g))) * f32(u)) over a row [g | u] of the
//                   fused gate+up output (cider/fused_hybrid.py:209), then q, sa
//                   silu(g) = g / (1 + exp(-g)) in fp32.
//   qk_norm_rope    per token and head of a fused q/k/v projection: RMSNorm of
//                   q and k over head_dim (own weights), rotate-half RoPE
//                   (q*cos + rot(q)*sin, each product and the sum rounded to
//                   fp16), q to a [L, H, D] buffer, k and v straight into the
//                   KV caches (both [KV, T, D]).
//
// The quantization of y is exactly the library's quantize_per_token applied to
// the fp16 y this kernel produces (same helpers), so q and sa are bit-identical
// to the unfused pair of calls on that y.  The RMSNorm and SiLU steps are the
// model's, not the reference library's; their fp32 sums run in a fixed order
// (each lane in element order, then an xor butterfly over the wave, then the
// waves in order when a workgroup shares a row).
//
// MI355X design: one 64-lane wave per row, 4 rows per workgroup.  A row of up
// to 64 * 32 * 8 = 16384 elements stays in registers (NV 16-byte vectors per
// lane) from the read through the reductions to the quantized store, so x is
// read from HBM once and only q (1 byte/element) and sa go back; longer rows
// stream from L2 a second and third time.  Reductions are wave-local
// (shuffles, no LDS, no barrier).  With at most 64 rows (decode) a row gets a
// whole 256-thread workgroup instead (four waves, LDS for the cross-wave sum
// and max); SwiGLU + quantize takes a workgroup per row at every M (rows of up
// to 16384 elements), and SwiGLU without quantization is elementwise over the
// grid.
#include "common.hpp"
#include "kernels.hpp"
#include "norm_common.hpp"
#include "quant_common.hpp"

namespace cider {

namespace {

// ---------------------------------------------------------------------------
// RMSNorm (+ residual add) (+ per-token quantize)
// ---------------------------------------------------------------------------
template <int NV, bool ADD, bool WY, bool WQ>
__global__ __launch_bounds__(256) void rmsnorm_kernel(
    const uint16_t* x, const uint16_t* __restrict__ add, uint16_t* hsum,
    const uint16_t* __restrict__ w, float eps, uint16_t* __restrict__ y,
    int8_t* __restrict__ q, float* __restrict__ sa, int M, int K) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;  // uniform per wave
  const int nvec = K >> 3;
  const uint16_t* xr = x + row * K;
  // h of vector e; with ADD the first pass writes it to hsum (which may alias x)
  auto first_h = [&](int e) -> i32x4 {
    i32x4 h = ld16(xr + 8 * e);
    if constexpr (ADD) {
      h = add8(h, ld16(add + row * K + 8 * e));
      *reinterpret_cast<i32x4*>(hsum + row * K + 8 * e) = h;
    }
    return h;
  };
  const uint16_t* hr = ADD ? hsum + row * K : xr;

  float ss = 0.0f, amax = 0.0f;
  if constexpr (NV > 0) {
    // up to 12 vectors per lane every load first, unconditional (clamped: a
    // lane past the row re-reads its last vector): a load under a lane mask
    // made the compiler wait for each before the next.  hsum may alias x:
    // each element's h is stored after all of the row's x loads, by the lane
    // that loaded it.  From 16 on the three register copies would not fit.
    constexpr bool HOIST = NV <= 12;
    i32x4 v[NV], av[HOIST && ADD ? NV : 1], wv[HOIST ? NV : 1];
    if constexpr (HOIST) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = min(lane + i * kWave, nvec - 1);
        v[i] = ld16(xr + 8 * e);
        if constexpr (ADD) av[i] = ld16(add + row * K + 8 * e);
        wv[i] = ld16(w + 8 * e);
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + i * kWave;
      if constexpr (HOIST) {
        if constexpr (ADD) {
          v[i] = add8(v[i], av[i]);
          if (e < nvec) *reinterpret_cast<i32x4*>(hsum + row * K + 8 * e) = v[i];
        }
        if (e >= nvec) v[i] = i32x4{0, 0, 0, 0};
      } else {
        v[i] = e < nvec ? first_h(e) : i32x4{0, 0, 0, 0};
      }
      ss = sumsq8(v[i], ss);
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + i * kWave;
      if (e < nvec) {
        if constexpr (HOIST)
          v[i] = norm8(v[i], wv[i], r);
        else
          v[i] = norm8(v[i], ld16(w + 8 * e), r);
        if constexpr (WY) *reinterpret_cast<i32x4*>(y + row * K + 8 * e) = v[i];
        amax = absmax8(v[i], amax);
      }
    }
    if constexpr (WQ) {
      amax = wave_max(amax);
      const float s = row_scale(amax);
      const float inv = 1.0f / s;
      if (lane == 0) sa[row] = s;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = lane + i * kWave;
        if (e < nvec) *reinterpret_cast<i32x2*>(q + row * K + 8 * e) = quant8(v[i], inv);
      }
    }
  } else {
    for (int e = lane; e < nvec; e += kWave) ss = sumsq8(first_h(e), ss);
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)K + eps);
    for (int e = lane; e < nvec; e += kWave) {
      const i32x4 v = norm8(ld16(hr + 8 * e), ld16(w + 8 * e), r);
      if constexpr (WY) *reinterpret_cast<i32x4*>(y + row * K + 8 * e) = v;
      amax = absmax8(v, amax);
    }
    if constexpr (WQ) {
      amax = wave_max(amax);
      const float s = row_scale(amax);
      const float inv = 1.0f / s;
      if (lane == 0) sa[row] = s;
      for (int e = lane; e < nvec; e += kWave)
        *reinterpret_cast<i32x2*>(q + row * K + 8 * e) =
            quant8(norm8(ld16(hr + 8 * e), ld16(w + 8 * e), r), inv);
    }
  }
}

// ---------------------------------------------------------------------------
// SwiGLU (+ per-token quantize)
// ---------------------------------------------------------------------------
// Rows above 16384 elements (the shorter ones take silu_mul_row_kernel): one
// wave per row, 4 rows per workgroup, the row streamed from L2 a second time
// for the quantized store.
template <bool WY, bool WQ>
__global__ __launch_bounds__(256) void silu_mul_kernel(
    const uint16_t* __restrict__ gu, uint16_t* __restrict__ y, int8_t* __restrict__ q,
    float* __restrict__ sa, int M, int I) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int nvec = I >> 3;
  const uint16_t* g = gu + row * 2 * I;
  const uint16_t* u = g + I;
  float amax = 0.0f;
  for (int e = lane; e < nvec; e += kWave) {
    const i32x4 v = swiglu8(ld16(g + 8 * e), ld16(u + 8 * e));
    if constexpr (WY) *reinterpret_cast<i32x4*>(y + row * I + 8 * e) = v;
    amax = absmax8(v, amax);
  }
  if constexpr (WQ) {
    amax = wave_max(amax);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (lane == 0) sa[row] = s;
    for (int e = lane; e < nvec; e += kWave)
      *reinterpret_cast<i32x2*>(q + row * I + 8 * e) =
          quant8(swiglu8(ld16(g + 8 * e), ld16(u + 8 * e)), inv);
  }
}

// ---------------------------------------------------------------------------
// Few rows (decode): one 256-thread workgroup per row, so a row's loads come
// from four waves at once; the sums and maxima go through LDS in wave order.
// ---------------------------------------------------------------------------
template <int NVB, bool ADD, bool WY, bool WQ>
__global__ __launch_bounds__(256) void rmsnorm_row_kernel(
    const uint16_t* x, const uint16_t* __restrict__ add, uint16_t* hsum,
    const uint16_t* __restrict__ w, float eps, uint16_t* __restrict__ y,
    int8_t* __restrict__ q, float* __restrict__ sa, int K) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int nvec = K >> 3;
  const uint16_t* xr = x + row * K;
  i32x4 v[NVB];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int e = tid + i * 256;
    if (e < nvec) {
      v[i] = ld16(xr + 8 * e);
      if constexpr (ADD) {
        v[i] = add8(v[i], ld16(add + row * K + 8 * e));
        *reinterpret_cast<i32x4*>(hsum + row * K + 8 * e) = v[i];
      }
    } else {
      v[i] = i32x4{0, 0, 0, 0};
    }
    ss = sumsq8(v[i], ss);
  }
  ss = block_sum4(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)K + eps);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int e = tid + i * 256;
    if (e < nvec) {
      v[i] = norm8(v[i], ld16(w + 8 * e), r);
      if constexpr (WY) *reinterpret_cast<i32x4*>(y + row * K + 8 * e) = v[i];
      amax = absmax8(v[i], amax);
    }
  }
  if constexpr (WQ) {
    amax = block_max4(amax, red);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (tid == 0) sa[row] = s;
#pragma unroll
    for (int i = 0; i < NVB; ++i) {
      const int e = tid + i * 256;
      if (e < nvec) *reinterpret_cast<i32x2*>(q + row * K + 8 * e) = quant8(v[i], inv);
    }
  }
}

template <int NVB, bool WY>
__global__ __launch_bounds__(256) void silu_mul_row_kernel(
    const uint16_t* __restrict__ gu, uint16_t* __restrict__ y, int8_t* __restrict__ q,
    float* __restrict__ sa, int I) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int nvec = I >> 3;
  const uint16_t* g = gu + row * 2 * I;
  const uint16_t* u = g + I;
  i32x4 v[NVB];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int e = tid + i * 256;
    if (e < nvec) {
      v[i] = swiglu8(ld16(g + 8 * e), ld16(u + 8 * e));
      if constexpr (WY) *reinterpret_cast<i32x4*>(y + row * I + 8 * e) = v[i];
      amax = absmax8(v[i], amax);
    }
  }
  amax = block_max4(amax, red);
  const float s = row_scale(amax);
  const float inv = 1.0f / s;
  if (tid == 0) sa[row] = s;
#pragma unroll
  for (int i = 0; i < NVB; ++i) {
    const int e = tid + i * 256;
    if (e < nvec) *reinterpret_cast<i32x2*>(q + row * I + 8 * e) = quant8(v[i], inv);
  }
}

// SwiGLU without quantization: no row reduction, one 8-element vector per
// thread over the whole [M, I] output.
__global__ __launch_bounds__(256) void silu_mul_ew_kernel(const uint16_t* __restrict__ gu,
                                                          uint16_t* __restrict__ y, int64_t M,
                                                          int I) {
  const int nvec = I >> 3;
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= M * nvec) return;
  const int64_t row = v / nvec;
  const int e = (int)(v % nvec);
  const uint16_t* g = gu + row * 2 * I;
  *reinterpret_cast<i32x4*>(y + row * I + 8 * e) = swiglu8(ld16(g + 8 * e), ld16(g + I + 8 * e));
}

// ---------------------------------------------------------------------------
// per-head q/k RMSNorm + RoPE + KV-cache write (head_dim 128)
// ---------------------------------------------------------------------------
// Eight lanes per (token, head) of the fused projection row [q heads | k
// heads | v heads], eight heads per wave: lane j of a head holds elements
// [8j, 8j + 8) and [64 + 8j, 64 + 8j + 8), which are the pairs the
// rotate-half RoPE mixes, so every access is 16 bytes.  The head's sum of
// squares: each lane's 16 squares in order, then pairs, quads and the 8-lane
// group by DPP moves.  Per element: n = h(w * h(x * r)), out = h(h(n * cos) +
// h(-n' * sin)) for the first half (n' its partner) and h(h(n * cos) +
// h(n' * sin)) for the second.  (One wave per head with 2-byte lanes ran the
// 2048-token prefill's 2048 x 48 heads in 29.5 us per call; this layout in
// 15.6 us.)
__device__ __forceinline__ float group8_sum(float v) {
  v = v + __builtin_bit_cast(float, dpp_mov<kDppXor1>(__builtin_bit_cast(int32_t, v)));
  v = v + __builtin_bit_cast(float, dpp_mov<kDppXor2>(__builtin_bit_cast(int32_t, v)));
  v = v + __builtin_bit_cast(float, dpp_mov<kDppMirror8>(__builtin_bit_cast(int32_t, v)));
  return v;
}

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, float eps, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int64_t P, const int64_t* __restrict__ rope_row,
    const int64_t* __restrict__ slot, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int L, int H, int KV, int64_t T) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63, j = lane & 7;
  const int heads = H + 2 * KV;
  const int groups = (heads + 7) / 8;  // waves per token
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t t = gw / groups;
  if (t >= L) return;  // uniform per wave
  const int hh = (int)(gw % groups) * 8 + (lane >> 3);
  if (hh >= heads) return;
  const uint16_t* src = qkv + (t * heads + hh) * D;
  const i32x4 x0 = ld16(src + 8 * j), x1 = ld16(src + 64 + 8 * j);
  const int64_t p = slot[t];
  if (hh >= H + KV) {  // v: copy into the cache
    if (p < 0 || p >= T) return;
    uint16_t* dst = vc + ((int64_t)(hh - H - KV) * T + p) * D;
    *reinterpret_cast<i32x4*>(dst + 8 * j) = x0;
    *reinterpret_cast<i32x4*>(dst + 64 + 8 * j) = x1;
    return;
  }
  const int64_t rr = rope_row[t];
  const bool has_row = rr >= 0 && rr < P;
  const uint16_t* wn = hh < H ? qw : kw;
  const int64_t rrc = has_row ? rr : 0;
  const i32x4 w0 = ld16(wn + 8 * j), w1 = ld16(wn + 64 + 8 * j);
  const i32x4 c0 = ld16(cos_t + rrc * D + 8 * j), c1 = ld16(cos_t + rrc * D + 64 + 8 * j);
  const i32x4 s0 = ld16(sin_t + rrc * D + 8 * j), s1 = ld16(sin_t + rrc * D + 64 + 8 * j);
  float ss = 0.0f;
  ss = sumsq8(x0, ss);
  ss = sumsq8(x1, ss);
  ss = group8_sum(ss);  // every lane of the head's group
  if (!has_row) {
    // No RoPE row: the k cache is left alone, and the q heads get a quiet
    // NaN, so a caller that feeds them on sees the error instead of stale
    // memory.
    if (hh < H) {
      uint16_t* dst = q_out + (t * H + hh) * D;
      const i32x4 nan4 = {0x7E007E00, 0x7E007E00, 0x7E007E00, 0x7E007E00};
      *reinterpret_cast<i32x4*>(dst + 8 * j) = nan4;
      *reinterpret_cast<i32x4*>(dst + 64 + 8 * j) = nan4;
    }
    return;
  }
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  const i32x4 n0 = norm8(x0, w0, r), n1 = norm8(x1, w1, r);
  i32x4 o0, o1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint16_t lo[2], hi[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float a = h2f(h ? hi16(n0[e]) : lo16(n0[e]));
      const float b = h2f(h ? hi16(n1[e]) : lo16(n1[e]));
      const float ca = h2f(h ? hi16(c0[e]) : lo16(c0[e]));
      const float sa = h2f(h ? hi16(s0[e]) : lo16(s0[e]));
      const float cb = h2f(h ? hi16(c1[e]) : lo16(c1[e]));
      const float sb = h2f(h ? hi16(s1[e]) : lo16(s1[e]));
      // out = x * cos + rotate_half(x) * sin, rotate_half(x) = [-x[64:], x[:64]]
      lo[h] = f2h(h2f(f2h(a * ca)) + h2f(f2h(-(b * sa))));
      hi[h] = f2h(h2f(f2h(b * cb)) + h2f(f2h(a * sb)));
    }
    o0[e] = pack2(lo[0], lo[1]);
    o1[e] = pack2(hi[0], hi[1]);
  }
  uint16_t* dst;
  if (hh < H) {
    dst = q_out + (t * H + hh) * D;
  } else {
    if (p < 0 || p >= T) return;
    dst = kc + ((int64_t)(hh - H) * T + p) * D;
  }
  *reinterpret_cast<i32x4*>(dst + 8 * j) = o0;
  *reinterpret_cast<i32x4*>(dst + 64 + 8 * j) = o1;
}

template <template <int> class F, typename... A>
hipError_t by_nv(int nvec, A... args) {
  const int per_lane = (nvec + kWave - 1) / kWave;
  if (per_lane <= 1) return F<1>::run(args...);
  if (per_lane <= 2) return F<2>::run(args...);
  if (per_lane <= 4) return F<4>::run(args...);
  if (per_lane <= 8) return F<8>::run(args...);
  if (per_lane <= 12) return F<12>::run(args...);
  if (per_lane <= 16) return F<16>::run(args...);
  if (per_lane <= 24) return F<24>::run(args...);
  if (per_lane <= 32) return F<32>::run(args...);
  return F<0>::run(args...);
}

template <int NV>
struct RmsRun {
  static hipError_t run(const uint16_t* x, const uint16_t* add, uint16_t* hsum,
                        const uint16_t* w, float eps, uint16_t* y, int8_t* q, float* sa,
                        int M, int K, hipStream_t s) {
    const dim3 grid((M + 3) / 4), block(256);
    const int sel = (add ? 4 : 0) | (y ? 2 : 0) | (q ? 1 : 0);
#define CIDER_RMS(A, Y, Q)                                                            \
  case (A ? 4 : 0) | (Y ? 2 : 0) | (Q ? 1 : 0):                                       \
    rmsnorm_kernel<NV, A, Y, Q><<<grid, block, 0, s>>>(x, add, hsum, w, eps, y, q, sa, \
                                                       M, K);                         \
    break;
    switch (sel) {
      CIDER_RMS(false, false, true)
      CIDER_RMS(false, true, false)
      CIDER_RMS(false, true, true)
      CIDER_RMS(true, false, true)
      CIDER_RMS(true, true, false)
      CIDER_RMS(true, true, true)
      default:
        return hipErrorInvalidValue;
    }
#undef CIDER_RMS
    return hipGetLastError();
  }
};

hipError_t run_swi_wave(const uint16_t* gu, uint16_t* y, int8_t* q, float* sa, int M, int I,
                        hipStream_t s) {
  const dim3 grid((M + 3) / 4), block(256);
  if (y && q)
    silu_mul_kernel<true, true><<<grid, block, 0, s>>>(gu, y, q, sa, M, I);
  else if (y)
    silu_mul_kernel<true, false><<<grid, block, 0, s>>>(gu, y, q, sa, M, I);
  else if (q)
    silu_mul_kernel<false, true><<<grid, block, 0, s>>>(gu, y, q, sa, M, I);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

namespace {

// rows at or below this count run one workgroup per row
constexpr int kFewRows = 64;

template <int NVB>
hipError_t run_rms_row(const uint16_t* x, const uint16_t* add, uint16_t* hsum, const uint16_t* w,
                       float eps, uint16_t* y, int8_t* q, float* sa, int M, int K, hipStream_t s) {
  const int sel = (add ? 4 : 0) | (y ? 2 : 0) | (q ? 1 : 0);
#define CIDER_RMSR(A, Y, Q)                                                              \
  case (A ? 4 : 0) | (Y ? 2 : 0) | (Q ? 1 : 0):                                          \
    rmsnorm_row_kernel<NVB, A, Y, Q><<<M, 256, 0, s>>>(x, add, hsum, w, eps, y, q, sa, K); \
    break;
  switch (sel) {
    CIDER_RMSR(false, false, true)
    CIDER_RMSR(false, true, false)
    CIDER_RMSR(false, true, true)
    CIDER_RMSR(true, false, true)
    CIDER_RMSR(true, true, false)
    CIDER_RMSR(true, true, true)
    default:
      return hipErrorInvalidValue;
  }
#undef CIDER_RMSR
  return hipGetLastError();
}

template <int NVB>
hipError_t run_swi_row(const uint16_t* gu, uint16_t* y, int8_t* q, float* sa, int M, int I,
                       hipStream_t s) {
  if (y)
    silu_mul_row_kernel<NVB, true><<<M, 256, 0, s>>>(gu, y, q, sa, I);
  else
    silu_mul_row_kernel<NVB, false><<<M, 256, 0, s>>>(gu, y, q, sa, I);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* add, uint16_t* hsum,
                          const uint16_t* w, float eps, uint16_t* y, int8_t* q, float* sa, int M,
                          int K, hipStream_t s) {
  const int nvec = K >> 3;
  if (M <= kFewRows) {
    if (nvec <= 256) return run_rms_row<1>(x, add, hsum, w, eps, y, q, sa, M, K, s);
    if (nvec <= 512) return run_rms_row<2>(x, add, hsum, w, eps, y, q, sa, M, K, s);
    if (nvec <= 1024) return run_rms_row<4>(x, add, hsum, w, eps, y, q, sa, M, K, s);
    if (nvec <= 2048) return run_rms_row<8>(x, add, hsum, w, eps, y, q, sa, M, K, s);
  }
  return by_nv<RmsRun>(nvec, x, add, hsum, w, eps, y, q, sa, M, K, s);
}

hipError_t launch_silu_mul(const uint16_t* gu, uint16_t* y, int8_t* q, float* sa, int M, int I,
                           hipStream_t s) {
  const int nvec = I >> 3;
  if (!q) {
    const int64_t total = (int64_t)M * nvec;
    silu_mul_ew_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(gu, y, M, I);
    return hipGetLastError();
  }
  // A workgroup per row at every M, not only for few rows: its four waves load
  // a row at once, and at prefill sizes that beats a wave per row too (M=512
  // I=6144: 7.65 -> 4.88 us; M=1024: 8.21 -> 7.43 us; M=2048 I=12288: 28.6 ->
  // 23.0 us).  The same bits: the row's only reduction is a max.
  if (nvec <= 256) return run_swi_row<1>(gu, y, q, sa, M, I, s);
  if (nvec <= 512) return run_swi_row<2>(gu, y, q, sa, M, I, s);
  if (nvec <= 1024) return run_swi_row<4>(gu, y, q, sa, M, I, s);
  if (nvec <= 2048) return run_swi_row<8>(gu, y, q, sa, M, I, s);
  return run_swi_wave(gu, y, q, sa, M, I, s);
}

hipError_t launch_qk_norm_rope(const uint16_t* qkv, const uint16_t* qw, const uint16_t* kw,
                               float eps, const uint16_t* cos_t, const uint16_t* sin_t, int64_t P,
                               const int64_t* rope_row, const int64_t* slot, uint16_t* q_out,
                               uint16_t* kc, uint16_t* vc, int L, int H, int KV, int64_t T,
                               hipStream_t s) {
  const int64_t waves = (int64_t)L * ((H + 2 * KV + 7) / 8);
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  qk_norm_rope_kernel<<<grid, block, 0, s>>>(qkv, qw, kw, eps, cos_t, sin_t, P, rope_row, slot,
                                             q_out, kc, vc, L, H, KV, T);
  return hipGetLastError();
}

}  // namespace cider
