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
#define CIDER_OP_W4A8_REF 5

/* Library version (major*10000 + minor*100 + patch). */
int cider_version(void);

/* Message of the last error returned on the calling thread ("" if none). */
const char* cider_last_error(void);

/* Bytes of scratch the linear entry points need for the given problem
 * (quantized activations int8 [M,K] and per-token scales fp32 [M], each
 * 256-byte aligned; on shapes with few output tiles also the partial sums of
 * the split-K GEMM, S*M*N*4 bytes: int32 for CIDER_OP_PERCHANNEL, fp32 for
 * CIDER_OP_PERGROUP and CIDER_OP_W4A8_PERGROUP (group_size given). A smaller
 * workspace of at least the first two parts runs one pass over K instead:
 * per-channel with the same results, per-group within the same tolerance).
 * 0 when the call needs none (M <= 1 on the W8 paths).
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

/* Maximum scratch of cider_perchannel_linear_noalloc, in bytes (32 MiB:
 * M*K + 4*M rounded up to 256-byte pieces, e.g. M*K up to about 33.5M). */
#define CIDER_NOALLOC_SCRATCH_BYTES (32u << 20)

/* cider_perchannel_linear without a workspace argument, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference, whose
 * primitives allocate their temporaries through MLX. The quantized
 * activations and scales go to a scratch array the library holds in device
 * memory, one per GPU for the life of the process
 * (CIDER_NOALLOC_SCRATCH_BYTES); problems needing more return
 * CIDER_E_INVALID. The call allocates nothing. Every call on one GPU shares
 * that GPU's scratch: calls that overlap on one GPU (other streams, other
 * threads) race, so a caller must order them. Results are identical to
 * cider_perchannel_linear. */
int cider_perchannel_linear_noalloc(const void* x_f16, const int8_t* w_nk,
                                    const float* sw, const void* bias_f16,
                                    void* y_f16, int64_t M, int64_t N,
                                    int64_t K, void* stream);

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
 * D_g is the exact int32 sum of group g.  The M >= 2 GEMM kernels evaluate
 * the fp32 chain over the groups with fused multiply-adds
 * (acc = fma(f32(D_g), s, acc)) where every scale of a tile is finite and
 * below 2^64 (else that tile runs the chain above as written), and split K
 * into fp32 chains that are then added, on mid-M shapes with few tiles; the
 * fp16 outputs are within 1e-3 relative / 1 fp16 ulp of the chain above, or
 * within its fp32 error bound where the sum cancels.  The small-M kernels
 * (M <= 16, and M <= 64 on N < 8192) keep the chain above bit for bit.
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

/* W4A8 linear on weights in the reference W4 layout, one call:
 * packed_kn uint8 [K/2, N] (high nibble = even k, value = nibble - 8,
 * cider/ops.py:93-116), sw fp32 [N], no bias. The weights are repacked into
 * the caller's workspace (cider_workspace_bytes(CIDER_OP_W4A8_REF, ...):
 * the quantization scratch plus N*K/2 bytes), then the call proceeds as
 * cider_w4a8_linear; results are identical to cider_w4_repack_ref followed
 * by cider_w4a8_linear. A caller that reuses the weights saves the repack
 * (N*K bytes of traffic per call) by holding the repacked copy itself.
 * Replaces _cider_prim.w4a8_linear argument for argument
 * (csrc/src/prim_bindings.cpp:23-25, csrc/src/w4a8_primitive.mm:266-283). */
int cider_w4a8_linear_ref(const void* x_f16, const uint8_t* packed_kn,
                          const float* sw, void* y_f16, void* ws,
                          size_t ws_bytes, int64_t M, int64_t N, int64_t K,
                          void* stream);

/* W4A8 per-group linear (library W4 layout, fp16 scales [K/gs, N],
 * gs in {64,128}; bias fp16 [N] or NULL):
 *   acc = sum_g f32(f32(D_g) * f32(scale[g,n])); y = h(f32(acc*sa[m]) [+ bias])
 * No reference counterpart: the reference has no per-group W4. This is the
 * per-group flush of cider/kernels/pergroup_int8_gemm.metal:152-189 applied
 * to int4 weights, with the tolerance of cider_pergroup_linear on the large
 * grids (fma flush) and the split-K shapes; the other kernels keep the
 * chain bit for bit. */
int cider_w4a8_pergroup_linear(const void* x_f16, const uint8_t* w4_nk,
                               const void* scale_gn_f16, const void* bias_f16,
                               void* y_f16, void* ws, size_t ws_bytes,
                               int64_t M, int64_t N, int64_t K, int group_size,
                               void* stream);

/* ---- producers of the linear's input, and decode attention ------------
 * The reference library has no such kernels: its models (Qwen3 through
 * mlx-lm, cider/fused_hybrid.py:142-213) run RMSNorm, SwiGLU, RoPE and SDPA
 * as MLX ops and hand the fp16 result to the linear, which quantizes it
 * (cider/kernels/w8a8_quantize.metal:17-87). These entry points are those
 * callers on the GPU, with the quantization fused into the producer. */

/* RMSNorm of fp16 rows [M,K] with fp16 weight w [K]:
 *   h = x, or h = h(x + add) written to sum (sum may alias x) when add != NULL
 *   r = 1 / sqrt(sum_k f32(h)^2 / K + eps)
 *   y = h(f32(w) * f32(h(h * r)))            -> y_f16 [M,K] if y_f16 != NULL
 *   q, sa = quantize_per_token(y)            -> q [M,K], sa [M] if q != NULL
 * q and sa are bit-identical to cider_quantize_per_token on that y. At least
 * one of y / q; K % 8 == 0; fp16 arrays 16-byte aligned, q 8-byte aligned;
 * y must not alias x or sum. */
int cider_rmsnorm_quantize(const void* x_f16, const void* add_f16, void* sum_f16,
                           const void* w_f16, float eps, void* y_f16, int8_t* q,
                           float* sa, int64_t M, int64_t K, void* stream);

/* SwiGLU of the fused gate+up output gu [M, 2I] (gate first, as
 * cider/fused_hybrid.py:209 splits it):
 *   y = h(f32(h(g / (1 + exp(-g)))) * f32(u))   -> y_f16 [M,I] if non-NULL
 *   q, sa = quantize_per_token(y)               -> if q != NULL
 * I % 8 == 0; alignment as cider_rmsnorm_quantize. */
int cider_silu_mul_quantize(const void* gu_f16, void* y_f16, int8_t* q, float* sa,
                            int64_t M, int64_t I, void* stream);

/* Decode (M == 1) per-channel linear y = W8A8(x') with the producer of its
 * input x' run inside the linear's x staging, one launch instead of two:
 *   cider_rmsnorm_mv: x' = RMSNorm(h) as cider_rmsnorm_quantize's y, with
 *     h = x, or h = h(x + add) written to sum when add != NULL (sum must not
 *     overlap x or add: every workgroup reads them);
 *   cider_swiglu_mv: x' = SwiGLU of gate_up [2K] (gate first), as
 *     cider_silu_mul_quantize's y.
 * then y [N] exactly as cider_perchannel_linear at M == 1 (the fp16 MV) on
 * x'. Both are bit-identical to the pair of calls they replace (same per-
 * element formulas, same sum-of-squares order). The reference has no
 * counterpart: its models run the producer as an MLX op before the linear
 * (cider/fused_hybrid.py:142-213). Requires K % 256 == 0, K <= 16384 and
 * 16-byte aligned x / gate_up, w, add, sum, norm_w; else CIDER_E_UNSUPPORTED
 * (use the two calls). y must not overlap any input. */
int cider_rmsnorm_mv(const void* x_f16, const void* add_f16, void* sum_f16,
                     const void* norm_w_f16, float eps, const int8_t* w,
                     const float* scale_w, const void* bias_f16, void* y_f16,
                     int64_t N, int64_t K, void* stream);
int cider_swiglu_mv(const void* gate_up_f16, const int8_t* w, const float* scale_w,
                    const void* bias_f16, void* y_f16, int64_t N, int64_t K,
                    void* stream);

/* Per-head RMSNorm of q and k (weights [D]) and rotate-half RoPE on the rows
 * of a fused q/k/v projection qkv [L, (H + 2 KV) * D]:
 *   q_out [L, H, D]          <- RoPE(RMSNorm(q))
 *   k_cache[j, slot[t], :]   <- RoPE(RMSNorm(k_j))    (cache [KV, T, D])
 *   v_cache[j, slot[t], :]   <- v_j                   (cache [KV, T, D])
 * using rows rope_row[t] of the cos / sin tables [P, D] (fp16); RoPE is
 * out = h(h(x*cos) + h(rot(x)*sin)), rot(x) = [-x[D/2:], x[:D/2]].
 * rope_row and slot are int64 device arrays [L]; a token whose rope_row is
 * outside [0, P) gets quiet-NaN q heads and no k-cache write, and a slot
 * outside [0, T) writes nothing to the caches.
 * D must be 128. */
int cider_qk_norm_rope(const void* qkv_f16, const void* q_norm_w_f16,
                       const void* k_norm_w_f16, float eps, const void* cos_f16,
                       const void* sin_f16, int64_t P, const int64_t* rope_row,
                       const int64_t* slot, void* q_out_f16, void* k_cache_f16,
                       void* v_cache_f16, int64_t L, int64_t H, int64_t KV,
                       int64_t D, int64_t T, void* stream);

/* Bytes of workspace cider_attn_decode needs (fp32 per-chunk partials). */
size_t cider_attn_decode_workspace_bytes(int64_t H, int64_t T);

/* Single-query grouped-query attention over the caches written by
 * cider_qk_norm_rope: for query head h of KV head j = h / (H / KV),
 *   out[h] = sum_{t < n} softmax_t(scale * q[h] . K[j,t,:]) V[j,t,:]
 * in fp32, rounded to fp16 [H, D]. n = min(*n_valid, T) is read on the
 * device (int64), so a captured call serves a growing sequence. D == 128,
 * H / KV in {1, 2, 4, 8}, T % 8 == 0; ws 256-byte aligned. */
int cider_attn_decode(const void* q_f16, const void* k_cache_f16,
                      const void* v_cache_f16, const int64_t* n_valid, float scale,
                      void* ws, size_t ws_bytes, void* out_f16, int64_t H,
                      int64_t KV, int64_t D, int64_t T, void* stream);

/* Bytes of workspace cider_attn_prefill uses for a chunk of c queries over n
 * cache slots with H query heads: the fp32 partials of a launch that splits
 * its keys over several workgroups per query block (when the query blocks
 * alone would fill few CUs); 0 when it does not split. */
size_t cider_attn_prefill_workspace_bytes(int64_t c, int64_t n, int64_t H);

/* Causal grouped-query attention of a prefill chunk over the caches written
 * by cider_qk_norm_rope: the chunk's c queries q [c, H, D] sit at cache slots
 * n - c .. n - 1 (their keys already written), and for query i, head h of KV
 * head j = h / (H / KV),
 *   out[i, h] = sum_{t <= n - c + i} softmax_t(scale * q[i,h] . K[j,t,:]) V[j,t,:]
 * rounded to fp16 [c, H, D].  Replaces the reference's prefill call of MLX's
 * fused SDPA (cider/fused_hybrid.py:179-196); fp32 scores and accumulation,
 * probabilities rounded to fp16 for the P.V product.  ws (256-byte aligned)
 * of cider_attn_prefill_workspace_bytes lets a launch with few query blocks
 * split its keys; NULL or a smaller ws runs unsplit (results within the same
 * bar, not bit-identical).  With n_dev non-NULL (device int64) the length is
 * read on the device, clamped to [c, n], and n is its upper bound (it sizes
 * the split), so one captured call serves chunks at any cache offset.
 * D == 128, 1 <= c <= n <= T, H % KV == 0; q, the caches and out 16-byte
 * aligned; out and ws must not overlap the inputs. */
int cider_attn_prefill(const void* q_f16, const void* k_cache_f16,
                       const void* v_cache_f16, float scale, void* ws,
                       size_t ws_bytes, void* out_f16, int64_t c, int64_t n,
                       const int64_t* n_dev, int64_t H, int64_t KV, int64_t D,
                       int64_t T, void* stream);

/* Bytes of workspace cider_attn_prefill_quantize uses: the split partials of
 * cider_attn_prefill_workspace_bytes when the launch splits, else c * H * 256
 * (the fp16 output before its quantization); 0 for shapes it rejects. */
size_t cider_attn_prefill_quantize_workspace_bytes(int64_t c, int64_t n, int64_t H);

/* cider_attn_prefill with its output quantized per token for the o
 * projection: q_out int8 [c, H * D] and sa_out fp32 [c] are, bit for bit,
 * cider_quantize_per_token of the fp16 output cider_attn_prefill computes
 * with the same ws (the reference quantizes the o projection's input inside
 * its W8A8 linear, csrc/src/w8a8_primitive.mm:180-203, with
 * cider/kernels/w8a8_quantize.metal:33-86).  A launch that splits its keys
 * quantizes in the kernel that merges the parts, so the fp16 output never
 * goes through HBM; one that does not writes it into ws and quantizes it from
 * there.  ws (256-byte aligned, not overlapping the other buffers) of
 * cider_attn_prefill_quantize_workspace_bytes; at least c * H * 256 bytes
 * (which run one part).  H <= 128; otherwise as cider_attn_prefill (q_out
 * 16-byte aligned).  The reference has no fused attention; this entry serves
 * the same prefill call (cider/fused_hybrid.py:179-196) and the o projection
 * after it. */
int cider_attn_prefill_quantize(const void* q_f16, const void* k_cache_f16,
                                const void* v_cache_f16, float scale, void* ws,
                                size_t ws_bytes, int8_t* q_out, float* sa_out,
                                int64_t c, int64_t n, const int64_t* n_dev,
                                int64_t H, int64_t KV, int64_t D, int64_t T,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CIDER_HIP_H */
