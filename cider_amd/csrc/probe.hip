// Measurement probes for bench.py (libcider_probe.so; not part of the
// linear's interface and not called by cider_amd).  They time what the
// hardware itself sustains, as ceilings for the two roofline figures:
//
//   cider_probe_mfma  -- the int8 MFMA rate on register-resident operands:
//     every CU runs one workgroup of 8 waves (two per SIMD, as the GEMM's
//     256 x 256 tile), each wave `iters` rounds of MFMAs into the accumulators
//     of a 128 x 64 tile (the GEMM wave's), as 24 v_mfma_i32_32x32x32_i8 or
//     64 v_mfma_i32_16x16x64_i8 per round, from operand sets loaded from
//     `src` at entry.  No memory traffic
//     in the loop: the rate is bounded by the matrix cores and the clock the
//     part holds under that load.  Random bytes in `src` toggle the
//     multipliers as the GEMM's data does; zero bytes show the data-dependent
//     part.  Lane 0 of every wave records s_memtime (shader clock) and
//     s_memrealtime (100 MHz reference) at entry and exit, so the caller can
//     compute the shader clock the waves ran at.
//
//   cider_probe_read  -- one launch that reads `nbytes` (a multiple of 20480)
//     in the layout of the M == 1 MV (mv_stream_kernel<2, 5>): 4 waves per
//     workgroup, each wave 5 KB of consecutive bytes, lane l the 16-byte chunks
//     l, l + 64, ..., l + 256, all requested at entry; each wave xor-reduces
//     them and writes 4 bytes (the MV's two fp16 outputs).  No x staging, no
//     arithmetic: the read limit of a weight stream of that size in one
//     launch.  Non-temporal loads, as the MV's (the faster of the two cache
//     policies for a stream read once: 5.78 against 5.99 us for 26 MB).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int kSets = 3, kA = 2, kB = 4;  // operand sets; blocks along n and m (32 x 32)
constexpr int kSets16 = 2, kA16 = 4, kB16 = 8;  // the same wave tile in 16 x 16 blocks
constexpr int kWaveSrc = 24 * 1024;             // operand bytes per wave (the larger form)

// FORM 0: 24 v_mfma_i32_32x32x32_i8 per round (3 operand sets of 2 + 4
// fragments, 8 accumulator blocks); FORM 1: 64 v_mfma_i32_16x16x64_i8 per
// round (2 sets of 4 + 8 fragments, 32 blocks, X block outer), the same
// 128 x 64 wave tile.
template <int FORM>
__global__ __launch_bounds__(512, 1) void probe_mfma_kernel(const int8_t* __restrict__ src,
                                                            int iters,
                                                            long long* __restrict__ clocks,
                                                            int32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 8 + (threadIdx.x >> 6);  // global wave
  long long t0 = 0, r0 = 0;
  if (lane == 0) {
    t0 = (long long)__builtin_amdgcn_s_memtime();
    r0 = (long long)__builtin_amdgcn_s_memrealtime();
  }
  // operands: 16 bytes per lane and fragment, distinct per wave
  const i32x4* s4 = reinterpret_cast<const i32x4*>(src + (int64_t)gw * kWaveSrc);
  int32_t h = 0;
  if constexpr (FORM == 0) {
    i32x4 A[kSets][kA], B[kSets][kB];
#pragma unroll
    for (int s = 0; s < kSets; ++s) {
#pragma unroll
      for (int a = 0; a < kA; ++a) A[s][a] = s4[(s * (kA + kB) + a) * 64 + lane];
#pragma unroll
      for (int b = 0; b < kB; ++b) B[s][b] = s4[(s * (kA + kB) + kA + b) * 64 + lane];
    }
    i32x16 acc[kA][kB];
#pragma unroll
    for (int a = 0; a < kA; ++a)
#pragma unroll
      for (int b = 0; b < kB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int s = 0; s < kSets; ++s)
#pragma unroll
        for (int a = 0; a < kA; ++a)
#pragma unroll
          for (int b = 0; b < kB; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[s][a], B[s][b], acc[a][b], 0, 0, 0);
    }
#pragma unroll
    for (int a = 0; a < kA; ++a)
#pragma unroll
      for (int b = 0; b < kB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) h += acc[a][b][r];
  } else {
    i32x4 A[kSets16][kA16], B[kSets16][kB16];
#pragma unroll
    for (int s = 0; s < kSets16; ++s) {
#pragma unroll
      for (int a = 0; a < kA16; ++a) A[s][a] = s4[(s * (kA16 + kB16) + a) * 64 + lane];
#pragma unroll
      for (int b = 0; b < kB16; ++b) B[s][b] = s4[(s * (kA16 + kB16) + kA16 + b) * 64 + lane];
    }
    i32x4 acc[kA16][kB16];
#pragma unroll
    for (int a = 0; a < kA16; ++a)
#pragma unroll
      for (int b = 0; b < kB16; ++b) acc[a][b] = i32x4{0, 0, 0, 0};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int s = 0; s < kSets16; ++s)
#pragma unroll
        for (int b = 0; b < kB16; ++b)
#pragma unroll
          for (int a = 0; a < kA16; ++a)
            acc[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[s][a], B[s][b], acc[a][b], 0, 0, 0);
    }
#pragma unroll
    for (int a = 0; a < kA16; ++a)
#pragma unroll
      for (int b = 0; b < kB16; ++b) h += acc[a][b][0] + acc[a][b][1] + acc[a][b][2] + acc[a][b][3];
  }
  sink[gw * 64 + lane] = h;
  if (lane == 0) {
    const long long t1 = (long long)__builtin_amdgcn_s_memtime();
    const long long r1 = (long long)__builtin_amdgcn_s_memrealtime();
    clocks[gw * 4 + 0] = t0;
    clocks[gw * 4 + 1] = t1;
    clocks[gw * 4 + 2] = r0;
    clocks[gw * 4 + 3] = r1;
  }
}

constexpr int kReadWaveBytes = 5120, kReadChunks = 5;  // 64 lanes x 16 B x 5

__global__ __launch_bounds__(256) void probe_read_kernel(const int8_t* __restrict__ src,
                                                         int32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
  const i32x4* p = reinterpret_cast<const i32x4*>(src + (int64_t)gw * kReadWaveBytes);
  i32x4 v[kReadChunks];
#pragma unroll
  for (int c = 0; c < kReadChunks; ++c) v[c] = __builtin_nontemporal_load(&p[lane + 64 * c]);
  int32_t h = 0;
#pragma unroll
  for (int c = 0; c < kReadChunks; ++c) h ^= v[c][0] ^ v[c][1] ^ v[c][2] ^ v[c][3];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) h ^= __shfl_xor(h, o);
  if (lane == 0) sink[gw] = h;
}

}  // namespace

extern "C" {

// The MFMA probe on `grid` workgroups of 512 threads; form 0: 32 x 32 x 32,
// 1: 16 x 16 x 64.  src: at least grid * cider_probe_mfma_src_bytes() bytes;
// clocks: 4 * grid * 8 int64; sink: grid * 512 int32.  Returns 0, -1 for bad
// arguments, or the HIP error code of the launch.
int cider_probe_mfma(const int8_t* src, int form, int iters, long long* clocks, int32_t* sink,
                     int grid, void* stream) {
  if (iters < 1 || grid < 1 || (form != 0 && form != 1)) return -1;
  if (form == 0)
    probe_mfma_kernel<0><<<grid, 512, 0, (hipStream_t)stream>>>(src, iters, clocks, sink);
  else
    probe_mfma_kernel<1><<<grid, 512, 0, (hipStream_t)stream>>>(src, iters, clocks, sink);
  return (int)hipGetLastError();
}

// Operand bytes cider_probe_mfma reads per workgroup.
long long cider_probe_mfma_src_bytes(void) { return 8LL * kWaveSrc; }

// Integer operations of one round of one wave: 2 M N K of its MFMAs.
long long cider_probe_mfma_round_ops(int form) {
  return form == 0 ? 24LL * 2 * 32 * 32 * 32 : 64LL * 2 * 16 * 16 * 64;
}

// The read probe over nbytes (a multiple of 20480) of src; sink: nbytes /
// 5120 int32.
int cider_probe_read(const int8_t* src, long long nbytes, int32_t* sink, void* stream) {
  if (nbytes <= 0 || nbytes % (4 * kReadWaveBytes) != 0) return -1;
  const unsigned grid = (unsigned)(nbytes / (4 * kReadWaveBytes));
  probe_read_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(src, sink);
  return (int)hipGetLastError();
}

}  // extern "C"
