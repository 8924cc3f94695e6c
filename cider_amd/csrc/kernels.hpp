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

// Small-M GEMM as a weight stream (skinny_stream.hip): 1 <= M <= 64,
// K % 64 == 0, K <= 16384, N % 4 == 0, aligned operands.
bool skinny_stream_supported(const GemmArgs& a, int wf, int epi, int gs);
hipError_t launch_skinny_stream(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s);
// Small-M GEMM as a weight stream through LDS (skinny_dma.hip): 1 <= M <= 16,
// K % 512 == 0 and K >= 1536, N % 4 == 0 (per-group N % 8 == 0), aligned.
bool skinny_dma_supported(const GemmArgs& a, int wf, int epi, bool sw_half, int gs);
hipError_t launch_skinny_dma(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s);
// The earlier small-M kernel (skinny.hip), for shapes the stream kernel does
// not take.
hipError_t launch_skinny(const GemmArgs& a, int wf, int epi, bool sw_half, int gs,
                         hipStream_t s);
hipError_t launch_gemm_dma(const GemmArgs& a, int epi, int wf, hipStream_t s);
// Split-K per-channel GEMM for shapes with few tiles (gemm_dma.hip): K slices
// (1 = no split), the int32 partial bytes they need, and the launch (split
// tiles into `part`, then the summing dequant into a.y).
int splitk_ways(int M, int N, int K);
size_t splitk_bytes(int M, int N, int K);
hipError_t launch_gemm_splitk(const GemmArgs& a, int S, int32_t* part, hipStream_t s);
hipError_t launch_gemm_dma_pg(const GemmArgs& a, int gs, bool sw_half, int wf, hipStream_t s);
// Split-K per-group GEMM for mid-M shapes with few tiles (gemm_dma_pg.hip):
// K slices (1 = no split), the fp32 partial bytes they need, and the launch
// (slices into `part`, then their sum with the epilogue into a.y).
int pg_splitk_ways(int M, int N, int K, int gs);
size_t pg_splitk_bytes(int M, int N, int K, int gs);
hipError_t launch_gemm_pg_splitk(const GemmArgs& a, int gs, bool sw_half, int wf, int S,
                                 float* part, hipStream_t s);

// Decode-sized GEMV on quantized activations (1 <= M <= 4), gemv_q.hip.
bool gemv_q_supported(const GemmArgs& a, int wf, bool fused);
hipError_t launch_gemv_q(const GemmArgs& a, int wf, int epi, int gs, hipStream_t s);
// Same, on fp16 activations x [M, K] quantized per token inside the kernel
// (a.x and a.sa are ignored).
hipError_t launch_gemv_qx(const uint16_t* x, const GemmArgs& a, int wf, int epi, int gs,
                          hipStream_t s);

// M == 1 fp16-activation MV (per-channel when gs == 0, else per-group).
// M == 1 per-channel linear with a producer run in its x staging (gemv.hip):
// XM_NORM x' = RMSNorm(x); XM_ADDNORM h = x + add (written to hsum by one
// workgroup), x' = RMSNorm(h); XM_SWIGLU x = [gate | up] of 2K, x' = SwiGLU.
// Requires mv_producer_supported (K % 256 == 0, K <= 16384, 16-byte aligned).
enum { XM_PLAIN = 0, XM_NORM = 1, XM_ADDNORM = 2, XM_SWIGLU = 3 };
struct MvProducer {
  const uint16_t* add = nullptr;  // XM_ADDNORM
  uint16_t* hsum = nullptr;       // XM_ADDNORM: h = x + add
  const uint16_t* nw = nullptr;   // XM_NORM / XM_ADDNORM
  float eps = 0.0f;
};
// Streaming MV (mv_stream.hip): K in its table (1024 <= K <= 16384,
// K % 256 == 0), 16-byte aligned x and w, gs % 16 == 0.
bool mv_stream_supported(const void* x, const void* w, const void* sw, int K, int gs);
hipError_t launch_mv_stream(int xm, const uint16_t* x, const int8_t* w, const float* sw,
                            const uint16_t* bias, uint16_t* y, int N, int K, int gs,
                            const MvProducer& pp, hipStream_t s);
// The lane-order MV of gemv.hip alone (reproduces the reference's 32-lane
// order); launch_mv / launch_mv_producer use it where the streaming MV does
// not apply.
hipError_t launch_mv_lanes(const uint16_t* x, const int8_t* w, const float* sw,
                           const uint16_t* bias, uint16_t* y, int N, int K, int gs,
                           hipStream_t s);
bool mv_producer_supported(const void* x, const void* w, int K);
hipError_t launch_mv_producer(int xm, const uint16_t* x, const uint16_t* add, uint16_t* hsum,
                              const uint16_t* nw, float eps, const int8_t* w, const float* sw,
                              const uint16_t* bias, uint16_t* y, int N, int K, hipStream_t s);
hipError_t launch_mv(const uint16_t* x, const int8_t* w, const float* sw,
                     const uint16_t* bias, uint16_t* y, int N, int K, int gs,
                     hipStream_t s);

// Producer kernels (fused.hip): RMSNorm (+ residual add) and SwiGLU, each
// optionally ending in the per-token quantization; per-head q/k RMSNorm +
// RoPE + KV-cache write.
hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* add, uint16_t* hsum,
                          const uint16_t* w, float eps, uint16_t* y, int8_t* q, float* sa, int M,
                          int K, hipStream_t s);
hipError_t launch_silu_mul(const uint16_t* gu, uint16_t* y, int8_t* q, float* sa, int M, int I,
                           hipStream_t s);
hipError_t launch_qk_norm_rope(const uint16_t* qkv, const uint16_t* qw, const uint16_t* kw,
                               float eps, const uint16_t* cos_t, const uint16_t* sin_t, int64_t P,
                               const int64_t* rope_row, const int64_t* slot, uint16_t* q_out,
                               uint16_t* kc, uint16_t* vc, int L, int H, int KV, int64_t T,
                               hipStream_t s);

// Single-query attention over a KV cache (attn_decode.hip).
size_t attn_decode_ws_floats(int H, int64_t T);
hipError_t launch_attn_decode(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                              const int64_t* n, float scale, float* ws, uint16_t* out, int H,
                              int KV, int64_t T, hipStream_t s);

// Causal attention of a prefill chunk over the KV cache (attn_prefill.hip):
// c queries at cache slots n - c .. n - 1, D == 128, H % KV == 0 (n_dev: n
// read on the device, n its upper bound).  Launches
// that would fill few CUs split their keys over parts when ws holds
// attn_prefill_ws_floats(c, n, H) floats (nullptr / fewer: one part).
int attn_prefill_parts(int c, int n, int H);
size_t attn_prefill_ws_floats(int c, int n, int H);
hipError_t launch_attn_prefill(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                               uint16_t* out, float scale, float* ws, size_t ws_floats, int c,
                               int n, const int64_t* n_dev, int H, int KV, int64_t T,
                               hipStream_t s);
// The same attention with its output quantized per token (q int8 [c, H*128],
// sa fp32 [c]): split launches quantize in the merge, one-part launches write
// the fp16 output into ws and quantize it from there.  ws: at least
// attn_prefill_quant_ws_bytes(c, n, H) bytes, 256-byte aligned (c*H*256 bytes
// run one part).
size_t attn_prefill_quant_ws_bytes(int c, int n, int H);
hipError_t launch_attn_prefill_quant(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                                     int8_t* qo, float* sa, float scale, void* ws,
                                     size_t ws_bytes, int c, int n, const int64_t* n_dev, int H,
                                     int KV, int64_t T, hipStream_t s);

hipError_t launch_w4_repack_ref(const uint8_t* src_kn, uint8_t* dst_nk, int N,
                                int K, hipStream_t s);

}  // namespace cider
