/*
 * cider_hip.h - C ABI of libcider_hip.so, the MI355X (gfx950) implementation
 * of cider's fused  quantize -> int8 GEMM -> dequant  linear.
 *
 * Every entry point replaces one function of the reference's nanobind module
 * `_cider_prim` (csrc/src/prim_bindings.cpp:15-35) or one of the kernels its
 * primitives launch; the replaced symbol is cited above each declaration.
 *
 * Conventions (all entry points):
 *   - pointers are DEVICE pointers to dense row-major arrays; fp16 values are
 *     passed as `const void*` holding IEEE binary16 bit patterns;
 *   - `stream` is a hipStream_t (NULL = the default stream); work is enqueued
 *     asynchronously on it, as MLX enqueues work on its stream at mx.eval;
 *   - the return value is CIDER_OK (0) or a negative error code; the message
 *     of the last error on the calling thread is cider_last_error();
 *   - the library allocates nothing: scratch memory is the caller's `ws`
 *     buffer of at least cider_workspace_bytes(...) bytes;
 *   - M == 0 or N == 0 is a no-op that returns CIDER_OK.
 */
#ifndef CIDER_HIP_H
#define CIDER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes. CIDER_E_INVALID maps to Python ValueError (the reference
 * throws std::invalid_argument: csrc/src/w8a8_primitive.mm:257-262,
 * csrc/src/pergroup_primitive.mm:282-295); CIDER_E_HIP maps to RuntimeError
 * (std::runtime_error: csrc/src/w8a8_primitive.mm:98-102). */
#define CIDER_OK 0
#define CIDER_E_INVALID (-1)
#define CIDER_E_HIP (-2)
#define CIDER_E_UNSUPPORTED (-3)

/* Operation ids for cider_workspace_bytes. */
#define CIDER_OP_PERCHANNEL 1
#define CIDER_OP_PERGROUP 2
#define CIDER_OP_W4A8 3
#define CIDER_OP_W4A8_PERGROUP 4

/* Library version (major*10000 + minor*100 + patch). */
int cider_version(void);

/* Message of the last error returned on the calling thread ("" if none). */
const char* cider_last_error(void);

/* Bytes of scratch the linear entry points need for the given problem
 * (quantized activations int8 [M,K] and per-token scales fp32 [M], each
 * 256-byte aligned). 0 when the call needs none (M <= 1 on the W8 paths).
 * Replaces the per-call temporaries of csrc/src/w8a8_primitive.mm:184-188
 * and the global ScratchPool of csrc/src/w4a8_primitive.mm:40-76. */
size_t cider_workspace_bytes(int op, int64_t M, int64_t N, int64_t K,
                             int group_size);

/* Per-token symmetric int8 quantization of fp16 x [M,K]:
 *   s = max|x_m| / 127 (1 if 0), q = clamp(round_half_away(x * (1/s)), -128, 127)
 * writes q int8 [M,K] and sa fp32 [M].
 * Replaces kernel quantize_per_token (cider/kernels/w8a8_quantize.metal:17-87),
 * dispatched by csrc/src/w8a8_primitive.mm:191-202. */
int cider_quantize_per_token(const void* x_f16, int8_t* q, float* sa,
                             int64_t M, int64_t K, void* stream);

/* Raw int8 GEMM, C[M,N] = A[M,K] . B[N,K]^T in int32 (exact).
 * Replaces _cider_prim.int8_matmul_int32 (csrc/src/prim_bindings.cpp:31-33,
 * csrc/src/w8a8_primitive.mm:280-342). */
int cider_int8_matmul_int32(const int8_t* a, const int8_t* b_nk, int32_t* c,
                            int64_t M, int64_t N, int64_t K, void* stream);

/* Per-channel W8A8 linear, y fp16 [M,N]:
 *   M == 1 : y = h(sw[n] * sum_k f32(w[n,k]) f32(x[k]) + bias[n])  (fp16 MV)
 *   M >= 2 : quantize x, then y = h(f32(acc) * sa[m] * sw[n] + bias[n])
 * w int8 [N,K], sw fp32 [N], bias fp16 [N] or NULL (no add).
 * Replaces _cider_prim.perchannel_linear (csrc/src/prim_bindings.cpp:18-20,
 * csrc/src/w8a8_primitive.mm:137-276). */
int cider_perchannel_linear(const void* x_f16, const int8_t* w_nk,
                            const float* sw, const void* bias_f16,
                            void* y_f16, void* ws, size_t ws_bytes, int64_t M,
                            int64_t N, int64_t K, void* stream);

/* Per-channel GEMM on already-quantized activations (q int8 [M,K], sa fp32
 * [M]); any M >= 1. This is dispatch 2 of csrc/src/w8a8_primitive.mm:207-247
 * on its own, for callers that quantize once and reuse q (e.g. a fused
 * q/k/v projection). */
int cider_perchannel_gemm(const int8_t* q, const float* sa, const int8_t* w_nk,
                          const float* sw, const void* bias_f16, void* y_f16,
                          int64_t M, int64_t N, int64_t K, void* stream);

/* Per-group W8A8 linear; sw_gn fp32 [K/group_size, N], group_size in
 * {64,128,256}, K % group_size == 0.
 *   M == 1 : fp16 MV with per-group scales
 *   M >= 2 : acc = sum_g f32(f32(D_g) * sw[g,n]); y = h(f32(acc*sa[m]) + bias[n])
 * Replaces _cider_prim.pergroup_linear (csrc/src/prim_bindings.cpp:21-27,
 * csrc/src/pergroup_primitive.mm:138-312). The reference's unused
 * `new_bias` argument has no counterpart. */
int cider_pergroup_linear(const void* x_f16, const int8_t* w_nk,
                          const float* sw_gn, const void* bias_f16, void* y_f16,
                          void* ws, size_t ws_bytes, int64_t M, int64_t N,
                          int64_t K, int group_size, void* stream);

/* Repack the reference W4 layout into the library's W4 layout:
 *   src: uint8 [K/2, N]; element (k, n) is the high nibble of src[k/2, n]
 *        for even k and the low nibble for odd k, value = nibble - 8
 *        (cider/ops.py:93-116);
 *   dst: uint8 [N, K/2]; element (n, k) is the low nibble of dst[n, k/2] for
 *        even k and the high nibble for odd k, two's-complement int4.
 * No reference counterpart (the reference GEMM reads [K/2,N] directly,
 * cider/kernels/w4a8_matmul.metal:47-70); done once per weight. */
int cider_w4_repack_ref(const uint8_t* src_kn, uint8_t* dst_nk, int64_t N,
                        int64_t K, void* stream);

/* W4A8 linear with per-output-column fp32 scales and no bias, on weights in
 * the library layout (see cider_w4_repack_ref); always quantize + GEMM, M=1
 * included:  y = h(f32(f32(acc) * sa[m]) * sw[n]).
 * Replaces _cider_prim.w4a8_linear (csrc/src/prim_bindings.cpp:28-30,
 * csrc/src/w4a8_primitive.mm:175-283). */
int cider_w4a8_linear(const void* x_f16, const uint8_t* w4_nk, const float* sw,
                      void* y_f16, void* ws, size_t ws_bytes, int64_t M,
                      int64_t N, int64_t K, void* stream);

/* W4A8 per-group linear (library W4 layout, fp16 scales [K/gs, N],
 * gs in {64,128}; bias fp16 [N] or NULL):
 *   acc = sum_g f32(f32(D_g) * f32(scale[g,n])); y = h(f32(acc*sa[m]) [+ bias])
 * No reference counterpart: the reference has no per-group W4. This is the
 * per-group flush of cider/kernels/pergroup_int8_gemm.metal:152-189 applied
 * to int4 weights. */
int cider_w4a8_pergroup_linear(const void* x_f16, const uint8_t* w4_nk,
                               const void* scale_gn_f16, const void* bias_f16,
                               void* y_f16, void* ws, size_t ws_bytes,
                               int64_t M, int64_t N, int64_t K, int group_size,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CIDER_HIP_H */
