// Single-query (decode) attention over a KV cache, grouped-query heads.
//
//   for query head h = j * G + r of KV head j (G = H / KV):
//     s_t = scale * sum_d f32(q[h,d]) * f32(K[j,t,d])        t < n
//     o   = sum_t softmax(s)_t * f32(V[j,t,d])               -> fp16 [H, D]
// with both caches [KV, T, D] (position-major, 256 bytes per position); n,
// the number of valid positions, is read from device memory so a captured
// decode step replays unchanged while the sequence grows.  All arithmetic is
// fp32 (the reference's models call MLX's fused SDPA here, whose
// accumulation order is not specified; parity is against an fp32 softmax
// attention, within a tolerance).
//
// MI355X design (split-K "flash decoding"):
//   * the cache is cut into chunks of 128 positions; workgroup (chunk c, KV
//     head j) computes, for all G query heads of j at once, the chunk's
//     scores, its max m_c, sum l_c and unnormalised output o_c (fp32) and
//     writes them to a workspace; a second kernel merges the chunks with the
//     usual max-rescaling.  Each K / V byte is read once for all G heads.
//   * scores: a thread owns 8 consecutive positions and 8 of the 128
//     dimensions (one 16-byte K load per position); the 16 dimension slices
//     are summed through LDS.
//   * P.V: a thread owns 8 dimensions (one 16-byte V load per position) and
//     8 positions; the 16 position slices are summed through LDS.
//   * the grid covers the cache capacity T; chunks at or past n exit at once
//     (n is clamped to T).
//   * with more than 4 query heads per KV head, the heads are split over
//     several workgroups that each read that KV head's chunk.
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

namespace {

constexpr int kD = 128;      // head dimension
constexpr int kChunk = 128;  // positions per workgroup

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ void unpack8(i32x4 v, float (&f)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = h2f((uint16_t)((uint32_t)v[j] & 0xffffu));
    f[2 * j + 1] = h2f((uint16_t)((uint32_t)v[j] >> 16));
  }
}

// A workgroup serves G query heads of one KV head (G <= 4: the LDS slices
// below hold G * 8 KB); R = (H / KV) / G workgroups share a KV head.
// workspace layout per (head block y, chunk c): G * (kD + 2) floats:
// o_c[G][kD], m_c[G], l_c[G]
template <int G, int R>
__global__ __launch_bounds__(256) void attn_chunk_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int64_t* __restrict__ n_ptr, float scale,
    float* __restrict__ ws, int64_t T, int nchunk) {
  __shared__ float qs[G][kD];
  __shared__ float part[16][G][kChunk];  // dimension / position slices
  __shared__ float ps[G][kChunk];        // scores, then probabilities
  __shared__ float ml[G][2];

  const int c = blockIdx.x, y = blockIdx.y, j = y / R, tid = threadIdx.x;
  const int64_t nn = *n_ptr;
  const int64_t n = nn < T ? nn : T;
  const int64_t c0 = (int64_t)c * kChunk;
  if (c0 >= n) return;  // uniform: nothing of this chunk is valid

  // Issue every load of the chunk first (K for the scores, V for P.V: neither
  // depends on the other), so the chunk costs one memory latency.  Positions
  // past n (within T) are loaded and never used; 8-position groups wholly
  // past n re-load group 0 of the chunk (always valid).
  const int tq = tid & 15, dq = tid >> 4;  // scores: 8 positions x 8 dimensions
  const int dv = tid & 15, ts = tid >> 4;  // P.V: 8 dimensions x 8 positions
  const int64_t tk0 = c0 + 8 * tq, tv0 = c0 + 8 * ts;
  i32x4 kv[8], vv[8];
  {
    const uint16_t* kp = kc + ((int64_t)j * T + (tk0 < n ? tk0 : c0)) * kD + 8 * dq;
#pragma unroll
    for (int i = 0; i < 8; ++i) kv[i] = ld16(kp + (int64_t)i * kD);
    const uint16_t* vp = vc + ((int64_t)j * T + (tv0 < n ? tv0 : c0)) * kD + 8 * dv;
#pragma unroll
    for (int i = 0; i < 8; ++i) vv[i] = ld16(vp + (int64_t)i * kD);
  }
  for (int e = tid; e < G * kD; e += 256) qs[e / kD][e % kD] = h2f(q[(int64_t)y * G * kD + e]);
  __syncthreads();

  // ---- scores: thread (dq, tq) sums dimensions 8dq..8dq+7 for positions
  // c0 + 8tq .. +7
  {
    const int64_t t0 = tk0;
    float acc[G][8];
#pragma unroll
    for (int r = 0; r < G; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[r][i] = 0.0f;
    if (t0 < n) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float kf[8];  // dimensions 8dq .. 8dq + 7 of position t0 + i
        unpack8(kv[i], kf);
#pragma unroll
        for (int r = 0; r < G; ++r) {
#pragma unroll
          for (int jd = 0; jd < 8; ++jd) acc[r][i] = acc[r][i] + qs[r][8 * dq + jd] * kf[jd];
        }
      }
    }
#pragma unroll
    for (int r = 0; r < G; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) part[dq][r][8 * tq + i] = acc[r][i];
  }
  __syncthreads();
  for (int e = tid; e < G * kChunk; e += 256) {
    const int r = e / kChunk, t = e % kChunk;
    float s = 0.0f;
#pragma unroll
    for (int dq = 0; dq < 16; ++dq) s = s + part[dq][r][t];
    ps[r][t] = (c0 + t < n) ? s * scale : -INFINITY;
  }
  __syncthreads();

  // ---- chunk softmax statistics: wave w handles heads w, w + 4, ...
  {
    const int wave = tid >> 6, lane = tid & 63;
    for (int r = wave; r < G; r += 4) {
      const float a = ps[r][lane], b = ps[r][lane + 64];
      const float m = wave_max_f(fmaxf(a, b));  // finite: position c0 < n is valid
      const float pa = expf(a - m), pb = expf(b - m);
      ps[r][lane] = pa;
      ps[r][lane + 64] = pb;
      const float l = wave_sum_f(pa + pb);
      if (lane == 0) {
        ml[r][0] = m;
        ml[r][1] = l;
      }
    }
  }
  __syncthreads();

  // ---- P.V: thread (ts, dv) sums positions 8ts..8ts+7 for dimensions
  // 8dv..8dv+7
  {
    float acc[G][8];
#pragma unroll
    for (int r = 0; r < G; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[r][i] = 0.0f;
    const int64_t t0 = tv0;
    if (t0 < n) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (t0 + i >= n) break;  // invalid positions may hold anything
        float vf[8];
        unpack8(vv[i], vf);
#pragma unroll
        for (int r = 0; r < G; ++r) {
          const float p = ps[r][8 * ts + i];
#pragma unroll
          for (int d = 0; d < 8; ++d) acc[r][d] = acc[r][d] + p * vf[d];
        }
      }
    }
    __syncthreads();  // every thread is done reading ps before part is reused
#pragma unroll
    for (int r = 0; r < G; ++r)
#pragma unroll
      for (int d = 0; d < 8; ++d) part[ts][r][8 * dv + d] = acc[r][d];
  }
  __syncthreads();
  float* out = ws + ((int64_t)y * nchunk + c) * G * (kD + 2);
  for (int e = tid; e < G * kD; e += 256) {
    const int r = e / kD, d = e % kD;
    float o = 0.0f;
#pragma unroll
    for (int ts = 0; ts < 16; ++ts) o = o + part[ts][r][d];
    out[e] = o;
  }
  if (tid < G) {
    out[G * kD + tid] = ml[tid][0];
    out[G * kD + G + tid] = ml[tid][1];
  }
}

// One wave per query head merges the chunks that hold valid positions: lane c
// reads chunk c's max and sum (64 chunks per pass), then every lane
// accumulates its two output dimensions over the chunks with the weights
// broadcast from the owning lane.
template <int G>
__global__ __launch_bounds__(64) void attn_merge_kernel(const float* __restrict__ ws,
                                                        const int64_t* __restrict__ n_ptr,
                                                        uint16_t* __restrict__ out, int nchunk,
                                                        int64_t T) {
  const int h = blockIdx.x, lane = threadIdx.x;
  const int j = h / G, r = h % G;  // j: head block
  const int64_t nn = *n_ptr;
  const int64_t n = nn < T ? nn : T;
  const int nc = (int)((n + kChunk - 1) / kChunk);
  const int last = nc < nchunk ? nc : nchunk;
  uint16_t* o = out + (int64_t)h * kD;
  if (last <= 0) {
    o[lane] = 0;
    o[lane + 64] = 0;
    return;
  }
  const float* base = ws + (int64_t)j * nchunk * G * (kD + 2);
  constexpr int kStride = G * (kD + 2);
  float m = -INFINITY;
  for (int c = lane; c < last; c += 64) m = fmaxf(m, base[(int64_t)c * kStride + G * kD + r]);
  m = wave_max_f(m);
  float l = 0.0f, a0 = 0.0f, a1 = 0.0f;
  for (int c0 = 0; c0 < last; c0 += 64) {
    const int c = c0 + lane;
    float f = 0.0f;
    if (c < last) {
      const float* p = base + (int64_t)c * kStride;
      f = expf(p[G * kD + r] - m);
      l = l + f * p[G * kD + G + r];
    }
    const int cnt = last - c0 < 64 ? last - c0 : 64;
    int i = 0;
    for (; i + 4 <= cnt; i += 4) {  // four chunks' loads in flight
      float fi[4], x0[4], x1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float* p = base + (int64_t)(c0 + i + u) * kStride + r * kD;
        fi[u] = __shfl(f, i + u);
        x0[u] = p[lane];
        x1[u] = p[lane + 64];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a0 = a0 + fi[u] * x0[u];
        a1 = a1 + fi[u] * x1[u];
      }
    }
    for (; i < cnt; ++i) {
      const float* p = base + (int64_t)(c0 + i) * kStride + r * kD;
      const float fi = __shfl(f, i);
      a0 = a0 + fi * p[lane];
      a1 = a1 + fi * p[lane + 64];
    }
  }
  l = wave_sum_f(l);
  o[lane] = f2h(a0 / l);
  o[lane + 64] = f2h(a1 / l);
}

template <int G, int R>
hipError_t run_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const int64_t* n,
                    float scale, float* ws, uint16_t* out, int KV, int64_t T, hipStream_t s) {
  const int nchunk = (int)((T + kChunk - 1) / kChunk);
  attn_chunk_kernel<G, R><<<dim3(nchunk, KV * R), 256, 0, s>>>(q, kc, vc, n, scale, ws, T,
                                                                nchunk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  attn_merge_kernel<G><<<KV * R * G, 64, 0, s>>>(ws, n, out, nchunk, T);
  return hipGetLastError();
}

}  // namespace

size_t attn_decode_ws_floats(int H, int64_t T) {
  const int64_t nchunk = (T + kChunk - 1) / kChunk;
  return (size_t)(nchunk * H * (kD + 2));
}

hipError_t launch_attn_decode(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                              const int64_t* n, float scale, float* ws, uint16_t* out, int H,
                              int KV, int64_t T, hipStream_t s) {
  switch (H / KV) {
    case 1: return run_attn<1, 1>(q, kc, vc, n, scale, ws, out, KV, T, s);
    case 2: return run_attn<2, 1>(q, kc, vc, n, scale, ws, out, KV, T, s);
    case 4: return run_attn<4, 1>(q, kc, vc, n, scale, ws, out, KV, T, s);
    case 8: return run_attn<4, 2>(q, kc, vc, n, scale, ws, out, KV, T, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace cider
