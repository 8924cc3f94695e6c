// Host-side launchers of the gfx950 kernels (internal to libcider_hip.so).
// Each launcher checks nothing: capi.hip validates every argument first.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cider {

enum Epilogue { EPI_I32 = 0, EPI_PC = 1, EPI_PG = 2 };
enum WeightFormat { W_I8 = 0, W_I4 = 1 };

// Arguments of the GEMM kernels (tiled and skinny).
struct GemmArgs {
  const int8_t* x;        // quantized activations int8 [M, K]
  const void* w;          // int8 [N, K]  or  packed int4 [N, K/2]
  const float* sa;        // per-token scales fp32 [M]            (PC, PG)
  const void* sw;         // fp32 [N] (PC) | fp32 or fp16 [K/gs, N] (PG)
  const uint16_t* bias;   // fp16 [N] or nullptr (no add)
  void* y;                // fp16 [M, N] (PC, PG) or int32 [M, N] (I32)
  int M, N, K;
};

hipError_t launch_quantize(const uint16_t* x, int8_t* q, float* sa, int M,
                           int K, hipStream_t s);

// C = epilogue(x . w^T).  wf: W_I8 / W_I4; epi: Epilogue; sw_half: PG scales
// are fp16; gs: group size (PG only).
hipError_t launch_gemm(const GemmArgs& a, int wf, int epi, bool sw_half,
                       int gs, hipStream_t s);

// M == 1 fp16-activation MV (per-channel when gs == 0, else per-group).
hipError_t launch_mv(const uint16_t* x, const int8_t* w, const float* sw,
                     const uint16_t* bias, uint16_t* y, int N, int K, int gs,
                     hipStream_t s);

hipError_t launch_w4_repack_ref(const uint8_t* src_kn, uint8_t* dst_nk, int N,
                                int K, hipStream_t s);

}  // namespace cider
