// Building blocks of the LDS-DMA GEMM kernels (gemm_dma.hip, gemm_dma_pg.hip):
// the 32x32x32 int8 MFMA, the LDS row swizzle, the global -> LDS DMA issue,
// explicit vmcnt waits and the tile order.
#pragma once

#include "common.hpp"

namespace cider {

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// LDS slot of 16-byte chunk c in row r for rows of BK bytes.  The 16 lanes
// that LDS serves together read 16 consecutive rows at one chunk; XOR-ing the
// chunk with (r / (256 / BK)) mod (BK / 16) sends them to 16 distinct 16-byte
// bank groups of the 256-byte bank window.
template <int BK>
__device__ __forceinline__ int swz(int r) {
  return (r / (256 / BK)) % (BK / 16);
}

// 16 bytes per lane from global `src` to LDS at lds_base + 16 * lane
// (gfx950 global_load_lds_dwordx4).  Issued from inline asm, so the compiler
// neither tracks nor waits for it: the caller waits with wait_vmcnt.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(src), "s"(lds_base)
      : "memory", "m0");
}

// As dma16, from `base` + off: base is wave-uniform and held in scalar
// registers (the instruction's saddr form), off a per-lane 32-bit byte offset.
// A k-stage then advances the scalar base only, with no per-lane 64-bit
// address arithmetic in the k-loop.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(off), "s"(base), "s"(lds_base)
      : "memory", "m0");
}

// As dma16s with the non-temporal cache policy, for weight streams read once
// per launch.
__device__ __forceinline__ void dma16s_nt(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %0, %1 nt"
      :
      : "v"(off), "s"(base), "s"(lds_base)
      : "memory", "m0");
}

// Waits until at most N vector-memory loads of this wave are outstanding
// (they complete in order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

constexpr int kLdsBytes = 160 * 1024;  // gfx950 LDS per workgroup

// Tile (m0, n0) of region t of a grid of BM x BN tiles over columns
// [n_begin, n_end): tiles are taken in groups of GROUP_M tile rows, n-major
// inside a group, so consecutive tiles share weight columns in L2.
template <int BM, int BN>
__device__ __forceinline__ void tile_coords(int t, int M, int n_begin, int n_end, int& m0,
                                            int& n0) {
  constexpr int GROUP_M = 4;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (n_end - n_begin + BN - 1) / BN;
  const int per_group = GROUP_M * tiles_n;
  const int grp = t / per_group;
  const int first_m = grp * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  m0 = (first_m + (t % per_group) % gm) * BM;
  n0 = n_begin + ((t % per_group) / gm) * BN;
}

// Compute units of the current device (host; cached per device).
int num_cus();

}  // namespace cider
