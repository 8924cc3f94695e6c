// Device helpers shared by the gfx950 kernels of libcider_hip.so.
//
// Numerics contract of every kernel in this library:
//   * binary32 arithmetic rounds each operation (built with -ffp-contract=off,
//     no fast-math), so  a*b*c+d  is evaluated as ((a*b)*c)+d, four roundings;
//   * float division is IEEE correctly rounded (HIP's default);
//   * fp32 -> fp16 is round-to-nearest-even (v_cvt_f16_f32 in RNE mode);
//   * integer dot products are exact int32 (i8 MFMA / integer adds).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cider {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// fp32 -> fp16 of an already rounded binary32 value.  The empty asm makes f
// opaque: without it the backend may fold  f2h(a * b)  (or  f2h(a * b + c))
// into one v_fma_mixlo_f16, which rounds the exact product straight to fp16
// (one rounding) instead of to binary32 and then to fp16 (two roundings), and
// differs from the specified order at fp16 midpoints.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> fp16 (RNE), a in the low half, b in the high half: one
// v_cvt_pk_f16_f32 of the already rounded binary32 values.  gfx950 converts
// the two-wide vector whole, so no multiply folds into it and no empty asm is
// needed (the asm of f2h orders the conversion against LDS traffic, which
// costs the GEMM epilogues their overlap).
__device__ __forceinline__ uint32_t f2h2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}

// 16x16x64 int8 MFMA: C[i][j] += sum_k A[i][k] * B[k][j].
// Operand layout (64 lanes, 16 bytes each): lane l holds row i = l % 16 of A
// (column j = l % 16 of B) and one 16-byte slice of K selected by l / 16; the
// slice-to-K mapping is the same for A and B, so any consistent assignment of
// K elements to (l / 16, byte) pairs yields the exact dot product.
// Result layout: lane l, element r holds C[4 * (l / 16) + r][l % 16].
__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Lane moves within rows of 16 lanes by DPP (a VALU operand modifier, no LDS
// round trip as with __shfl_xor): lane l reads lane l ^ 1, l ^ 2, the mirror
// of l in its 8 lanes (7 - l) or in its 16 lanes (15 - l).
template <int CTRL>
__device__ __forceinline__ int32_t dpp_mov(int32_t v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppMirror8 = 0x141, kDppMirror16 = 0x140;

// Every lane of each aligned group of G lanes (G = 1, 2, 4, 8 or 16) gets the
// group's int32 sum (exact in any order).
template <int G>
__device__ __forceinline__ int32_t group_sum_i32(int32_t v) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "lane group");
  if constexpr (G >= 2) v += dpp_mov<kDppXor1>(v);
  if constexpr (G >= 4) v += dpp_mov<kDppXor2>(v);
  if constexpr (G >= 8) v += dpp_mov<kDppMirror8>(v);
  if constexpr (G >= 16) v += dpp_mov<kDppMirror16>(v);
  return v;
}

// Sum over the 64 lanes, in every lane: int32 (exact), and fp32 in a fixed
// order (pairs, quads, 8s and 16s by DPP; then the four 16-lane row sums,
// read into scalar registers, as (r0 + r1) + (r2 + r3)).
__device__ __forceinline__ int32_t wave_sum_i32(int32_t v) {
  v = group_sum_i32<16>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = v + __builtin_bit_cast(float, dpp_mov<kDppXor1>(__builtin_bit_cast(int32_t, v)));
  v = v + __builtin_bit_cast(float, dpp_mov<kDppXor2>(__builtin_bit_cast(int32_t, v)));
  v = v + __builtin_bit_cast(float, dpp_mov<kDppMirror8>(__builtin_bit_cast(int32_t, v)));
  v = v + __builtin_bit_cast(float, dpp_mov<kDppMirror16>(__builtin_bit_cast(int32_t, v)));
  const int32_t b = __builtin_bit_cast(int32_t, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// Sign-extends the four two's-complement nibbles held in the low half of each
// byte of t (t & 0xF0F0F0F0 == 0) to four int8 bytes, without carries between
// bytes:  (n ^ 0x88) - 8  lies in [120, 135] for every nibble n, and xor 0x80
// maps it to n - 16*(n >= 8) modulo 256.
__device__ __forceinline__ uint32_t sext_nibbles(uint32_t t) {
  return ((t ^ 0x88888888u) - 0x08080808u) ^ 0x80808080u;
}

// Unpacks one 32-bit word of packed int4 (byte j holds element 2j in its low
// nibble and 2j+1 in its high nibble) into 8 int8 values in element order:
// e0123 = elements 0..3, e4567 = elements 4..7.
__device__ __forceinline__ void unpack_w4_word(uint32_t w, uint32_t& e0123,
                                               uint32_t& e4567) {
  const uint32_t ev = sext_nibbles(w & 0x0F0F0F0Fu);         // elems 0,2,4,6
  const uint32_t od = sext_nibbles((w >> 4) & 0x0F0F0F0Fu);  // elems 1,3,5,7
  // v_perm_b32(S0=od, S1=ev): selector bytes 0-3 pick ev, 4-7 pick od.
  e0123 = __builtin_amdgcn_perm(od, ev, 0x05010400u);
  e4567 = __builtin_amdgcn_perm(od, ev, 0x07030602u);
}

// Loads `n` (< 16) bytes with byte loads, zero-filling the rest.
__device__ __forceinline__ i32x4 load_bytes_partial(const int8_t* p, int n) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  for (int i = 0; i < n; ++i)
    w[i >> 2] |= (uint32_t)(uint8_t)p[i] << (8 * (i & 3));
  return i32x4{(int32_t)w[0], (int32_t)w[1], (int32_t)w[2], (int32_t)w[3]};
}

__device__ __forceinline__ i32x4 ld16(const void* p) {
  return *reinterpret_cast<const i32x4*>(p);
}

__device__ __forceinline__ i32x2 ld8(const void* p) {
  return *reinterpret_cast<const i32x2*>(p);
}

// Non-temporal loads (the nt cache policy) for weight streams that every
// launch reads once: a single-launch read of 26 MB in the MV's layout ran
// 5.78 against 5.99 us with plain loads, the M == 1 MV 6.44 -> 6.00 us.
__device__ __forceinline__ i32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
}

__device__ __forceinline__ i32x2 ld8_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const i32x2*>(p));
}

// Maps a linear workgroup id to a tile index so that the workgroups one XCD
// runs (the hardware deals workgroups to the 8 XCDs round-robin) receive a
// contiguous range of tiles; neighbouring tiles share operand panels, which
// then hit in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int wg, int nwg) {
  constexpr int kXcd = 8;
  const int per = nwg / kXcd;          // full rounds
  const int full = per * kXcd;
  if (wg >= full) return wg;           // ragged tail keeps its id
  return (wg % kXcd) * per + wg / kXcd;
}

}  // namespace cider
