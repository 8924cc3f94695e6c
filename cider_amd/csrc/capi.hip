// extern "C" entry points of libcider_hip.so (declared in include/cider_hip.h).
//
// This layer is the counterpart of the reference's op constructors and
// primitive eval_gpu methods (csrc/src/w8a8_primitive.mm:137-342,
// csrc/src/pergroup_primitive.mm:138-312, csrc/src/w4a8_primitive.mm:175-283):
// it validates shapes and group sizes (std::invalid_argument there,
// CIDER_E_INVALID here), carves the quantized-activation scratch out of the
// caller's workspace, and applies the reference's dispatch policy:
//   W8 per-channel / per-group: M == 1 -> fp16 MV, otherwise quantize -> GEMM
//   W4A8: always quantize -> GEMM (M == 1 included)
// For decode-sized M (<= 4) "quantize -> GEMM" is one GEMV kernel that
// quantizes while staging x (identical q and scale_a).
// The GEMM launcher picks the tile shape from M (skinny for M <= 64); the
// choice never changes results on the integer path.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "cider_hip.h"
#include "kernels.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return CIDER_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess)
    return fail(CIDER_E_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return ok();
}

constexpr int64_t kMaxDim = (int64_t)1 << 30;

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

size_t quant_ws_bytes(int64_t M, int64_t K) {
  return align256((size_t)M * (size_t)K) + align256((size_t)M * sizeof(float));
}

int check_dims(const char* fn, int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0)
    return fail(CIDER_E_INVALID, "%s: negative dimension (M=%lld N=%lld K=%lld)", fn,
                (long long)M, (long long)N, (long long)K);
  if (M > kMaxDim || N > kMaxDim || K > kMaxDim)
    return fail(CIDER_E_INVALID, "%s: dimension above 2^30 (M=%lld N=%lld K=%lld)", fn,
                (long long)M, (long long)N, (long long)K);
  return CIDER_OK;
}

int need(const char* fn, const void* p, const char* name, bool required) {
  if (required && p == nullptr)
    return fail(CIDER_E_INVALID, "%s: %s is NULL", fn, name);
  return CIDER_OK;
}

#define CIDER_TRY(expr)           \
  do {                            \
    const int _rc = (expr);       \
    if (_rc != CIDER_OK) return _rc; \
  } while (0)

int check_ws(const char* fn, const void* ws, size_t ws_bytes, size_t needed) {
  if (needed == 0) return CIDER_OK;
  if (ws == nullptr)
    return fail(CIDER_E_INVALID, "%s: workspace is NULL (%zu bytes needed)", fn, needed);
  if (ws_bytes < needed)
    return fail(CIDER_E_INVALID, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, needed);
  if (((uintptr_t)ws & 255) != 0)
    return fail(CIDER_E_INVALID, "%s: workspace must be 256-byte aligned", fn);
  return CIDER_OK;
}

// Decode-sized calls run one GEMV kernel that quantizes x per token while
// staging it (same helpers as the quantize kernel, so the same q and scale_a)
// instead of a quantize launch followed by a GEMM launch: M == 1 (W4A8; the
// int8 formats run the fp16 MV there), and 2 <= M <= 4 while the quantization
// every 16-row workgroup repeats stays small (N / 16 * M * K <= 2^20
// elements).  Past that the repeated quantization costs more than the launch
// it saves: N=10240 K=2560 M=2 ran 13.3 us fused against 10.8 us as quantize
// + GEMV, M=4 24.9 against 13.3 us (W4A8 gs 128, N=12288 K=4096 M=4: 22.5
// against 15.0 us).  Returns true and the launch status in *rc if it ran.
bool try_fused_gemv(const char* fn, const void* x, const cider::GemmArgs& g, int wf, int epi,
                    int gs, hipStream_t s, int* rc) {
  cider::GemmArgs t = g;
  t.x = reinterpret_cast<const int8_t*>(x);
  if (!cider::gemv_q_supported(t, wf, true)) return false;
  if (g.M > 1 && (int64_t)((g.N + 15) / 16) * g.M * g.K > ((int64_t)1 << 20)) return false;
  *rc = hip_status(cider::launch_gemv_qx(reinterpret_cast<const uint16_t*>(x), g, wf, epi, gs, s),
                   fn);
  return true;
}

// Quantizes x into the workspace; returns q and sa pointers.
int quantize_into_ws(const char* fn, const void* x, void* ws, int64_t M, int64_t K,
                     hipStream_t s, int8_t** q, float** sa) {
  *q = reinterpret_cast<int8_t*>(ws);
  *sa = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + align256((size_t)M * (size_t)K));
  return hip_status(cider::launch_quantize(reinterpret_cast<const uint16_t*>(x), *q, *sa,
                                           (int)M, (int)K, s),
                    fn);
}

// ---- scratch of the entry points that allocate nothing --------------------
//
// One array per GPU, in the library's code object: it exists on every device
// the library is loaded on, until the process ends.  Host code must not use
// the name `scratch` as an address (it is a host-side stand-in); each
// device's address is read once with hipGetSymbolAddress, with that device
// current, and kept in scratch_dev[].
static __device__ __attribute__((aligned(256))) int8_t scratch[CIDER_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxDevices] = {};

// The current device's address of `scratch`.
int scratch_ptr(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, fn);
  if (dev < 0 || dev >= kMaxDevices)
    return fail(CIDER_E_UNSUPPORTED, "%s: device %d beyond the %d the library tracks", fn, dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, fn);
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return CIDER_OK;
}

}  // namespace

extern "C" {

int cider_version(void) { return 100; }  // 0.1.0

const char* cider_last_error(void) { return g_last_error.c_str(); }

size_t cider_workspace_bytes(int op, int64_t M, int64_t N, int64_t K, int group_size) {
  if (M <= 0 || K < 0) return 0;
  switch (op) {
    case CIDER_OP_PERCHANNEL:
      // quantized activations and scales, plus the int32 partial sums of the
      // split-K GEMM where that shape takes it
      if (M <= 1) return 0;
      if (N <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return quant_ws_bytes(M, K);
      return quant_ws_bytes(M, K) + align256(cider::splitk_bytes((int)M, (int)N, (int)K));
    case CIDER_OP_PERGROUP:
      // quantized activations and scales, plus the fp32 partial sums of the
      // split-K GEMM where that shape takes it
      if (M <= 1) return 0;
      if (N <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return quant_ws_bytes(M, K);
      return quant_ws_bytes(M, K) +
             align256(cider::pg_splitk_bytes((int)M, (int)N, (int)K, group_size));
    case CIDER_OP_W4A8:
      return quant_ws_bytes(M, K);
    case CIDER_OP_W4A8_PERGROUP:
      if (N <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return quant_ws_bytes(M, K);
      return quant_ws_bytes(M, K) +
             align256(cider::pg_splitk_bytes((int)M, (int)N, (int)K, group_size));
    case CIDER_OP_W4A8_REF:
      if (N < 0) return 0;
      return quant_ws_bytes(M, K) + align256((size_t)N * (size_t)(K / 2));
    default:
      return 0;
  }
}

int cider_quantize_per_token(const void* x_f16, int8_t* q, float* sa, int64_t M, int64_t K,
                             void* stream) {
  static const char* fn = "cider_quantize_per_token";
  CIDER_TRY(check_dims(fn, M, 1, K));
  if (M == 0) return ok();
  const bool elems = K > 0;
  CIDER_TRY(need(fn, x_f16, "x", elems));
  CIDER_TRY(need(fn, q, "q", elems));
  CIDER_TRY(need(fn, sa, "sa", true));
  return hip_status(cider::launch_quantize(reinterpret_cast<const uint16_t*>(x_f16), q, sa,
                                           (int)M, (int)K, (hipStream_t)stream),
                    fn);
}

int cider_int8_matmul_int32(const int8_t* a, const int8_t* b_nk, int32_t* c, int64_t M,
                            int64_t N, int64_t K, void* stream) {
  static const char* fn = "cider_int8_matmul_int32";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (M == 0 || N == 0) return ok();
  CIDER_TRY(need(fn, a, "a", K > 0));
  CIDER_TRY(need(fn, b_nk, "b", K > 0));
  CIDER_TRY(need(fn, c, "c", true));
  cider::GemmArgs g{a, b_nk, nullptr, nullptr, nullptr, c, (int)M, (int)N, (int)K};
  return hip_status(cider::launch_gemm(g, cider::W_I8, cider::EPI_I32, false, 0,
                                       (hipStream_t)stream),
                    fn);
}

int cider_perchannel_gemm(const int8_t* q, const float* sa, const int8_t* w_nk, const float* sw,
                          const void* bias_f16, void* y_f16, int64_t M, int64_t N, int64_t K,
                          void* stream) {
  static const char* fn = "cider_perchannel_gemm";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (M == 0 || N == 0) return ok();
  CIDER_TRY(need(fn, q, "q", K > 0));
  CIDER_TRY(need(fn, sa, "sa", true));
  CIDER_TRY(need(fn, w_nk, "w", K > 0));
  CIDER_TRY(need(fn, sw, "scale_w", true));
  CIDER_TRY(need(fn, y_f16, "y", true));
  cider::GemmArgs g{q, w_nk, sa, sw, reinterpret_cast<const uint16_t*>(bias_f16), y_f16,
                    (int)M, (int)N, (int)K};
  return hip_status(cider::launch_gemm(g, cider::W_I8, cider::EPI_PC, false, 0,
                                       (hipStream_t)stream),
                    fn);
}

int cider_perchannel_linear(const void* x_f16, const int8_t* w_nk, const float* sw,
                            const void* bias_f16, void* y_f16, void* ws, size_t ws_bytes,
                            int64_t M, int64_t N, int64_t K, void* stream) {
  static const char* fn = "cider_perchannel_linear";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (M == 0 || N == 0) return ok();
  CIDER_TRY(need(fn, x_f16, "x", K > 0));
  CIDER_TRY(need(fn, w_nk, "w", K > 0));
  CIDER_TRY(need(fn, sw, "scale_w", true));
  CIDER_TRY(need(fn, y_f16, "y", true));
  const hipStream_t s = (hipStream_t)stream;
  const uint16_t* bias = reinterpret_cast<const uint16_t*>(bias_f16);
  if (M == 1)
    return hip_status(cider::launch_mv(reinterpret_cast<const uint16_t*>(x_f16), w_nk, sw, bias,
                                       reinterpret_cast<uint16_t*>(y_f16), (int)N, (int)K, 0, s),
                      fn);
  CIDER_TRY(check_ws(fn, ws, ws_bytes, quant_ws_bytes(M, K)));
  int rc;
  const cider::GemmArgs gf{nullptr, w_nk, nullptr, sw, bias, y_f16, (int)M, (int)N, (int)K};
  if (try_fused_gemv(fn, x_f16, gf, cider::W_I8, cider::EPI_PC, 0, s, &rc)) return rc;
  int8_t* q;
  float* sa;
  CIDER_TRY(quantize_into_ws(fn, x_f16, ws, M, K, s, &q, &sa));
  cider::GemmArgs g{q, w_nk, sa, sw, bias, y_f16, (int)M, (int)N, (int)K};
  // Split-K where the shape takes it and the workspace holds the partial sums
  // (a workspace sized for the quantized activations alone runs one pass)
  const int S = cider::splitk_ways((int)M, (int)N, (int)K);
  const size_t qbytes = quant_ws_bytes(M, K);
  if (S > 1 && ws_bytes >= qbytes + cider::splitk_bytes((int)M, (int)N, (int)K) &&
      aligned16(w_nk) && aligned16(y_f16) && aligned16(sw) && aligned16(q)) {
    int32_t* part = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(ws) + qbytes);
    return hip_status(cider::launch_gemm_splitk(g, S, part, s), fn);
  }
  return hip_status(cider::launch_gemm(g, cider::W_I8, cider::EPI_PC, false, 0, s), fn);
}

int cider_perchannel_linear_noalloc(const void* x_f16, const int8_t* w_nk, const float* sw,
                                    const void* bias_f16, void* y_f16, int64_t M, int64_t N,
                                    int64_t K, void* stream) {
  static const char* fn = "cider_perchannel_linear_noalloc";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (M == 0 || N == 0) return ok();
  // the quantized activations and scales only (no split-K partial sums)
  const size_t need = M <= 1 ? 0 : quant_ws_bytes(M, K);
  if (need > (size_t)CIDER_NOALLOC_SCRATCH_BYTES)
    return fail(CIDER_E_INVALID,
                "%s: M=%lld K=%lld needs %zu bytes of scratch, above the library's %zu "
                "(M*K + 4*M, each 256-byte aligned); use cider_perchannel_linear with a "
                "workspace",
                fn, (long long)M, (long long)K, need, (size_t)CIDER_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) CIDER_TRY(scratch_ptr(fn, &ws));
  return cider_perchannel_linear(x_f16, w_nk, sw, bias_f16, y_f16, ws, need, M, N, K, stream);
}

namespace {

// The split-K partial sums of a per-group linear in the caller's workspace
// (after the quantized activations), when the shape takes the split and the
// workspace holds them; nullptr runs the one-pass GEMM (same contract, the
// sequential chain).
float* pg_splitk_part(const cider::GemmArgs& g, void* ws, size_t ws_bytes, int gs) {
  const int S = cider::pg_splitk_ways(g.M, g.N, g.K, gs);
  if (S <= 1) return nullptr;
  const size_t qbytes = quant_ws_bytes(g.M, g.K);
  if (ws_bytes < qbytes + cider::pg_splitk_bytes(g.M, g.N, g.K, gs)) return nullptr;
  if (!(aligned16(g.x) && aligned16(g.w) && aligned16(g.y) && aligned16(g.sw))) return nullptr;
  return reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + qbytes);
}

}  // namespace

int cider_pergroup_linear(const void* x_f16, const int8_t* w_nk, const float* sw_gn,
                          const void* bias_f16, void* y_f16, void* ws, size_t ws_bytes,
                          int64_t M, int64_t N, int64_t K, int group_size, void* stream) {
  static const char* fn = "cider_pergroup_linear";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (group_size != 64 && group_size != 128 && group_size != 256)
    return fail(CIDER_E_INVALID, "%s: group_size must be 64, 128, or 256 (got %d)", fn,
                group_size);
  if (K % group_size != 0)
    return fail(CIDER_E_INVALID, "%s: K=%lld is not a multiple of group_size=%d", fn,
                (long long)K, group_size);
  if (M == 0 || N == 0) return ok();
  CIDER_TRY(need(fn, x_f16, "x", K > 0));
  CIDER_TRY(need(fn, w_nk, "w", K > 0));
  CIDER_TRY(need(fn, sw_gn, "scale_w", K > 0));
  CIDER_TRY(need(fn, y_f16, "y", true));
  const hipStream_t s = (hipStream_t)stream;
  const uint16_t* bias = reinterpret_cast<const uint16_t*>(bias_f16);
  if (M == 1)
    return hip_status(cider::launch_mv(reinterpret_cast<const uint16_t*>(x_f16), w_nk, sw_gn,
                                       bias, reinterpret_cast<uint16_t*>(y_f16), (int)N, (int)K,
                                       group_size, s),
                      fn);
  CIDER_TRY(check_ws(fn, ws, ws_bytes, quant_ws_bytes(M, K)));
  int rc;
  const cider::GemmArgs gf{nullptr, w_nk, nullptr, sw_gn, bias, y_f16, (int)M, (int)N, (int)K};
  if (try_fused_gemv(fn, x_f16, gf, cider::W_I8, cider::EPI_PG, group_size, s, &rc)) return rc;
  int8_t* q;
  float* sa;
  CIDER_TRY(quantize_into_ws(fn, x_f16, ws, M, K, s, &q, &sa));
  cider::GemmArgs g{q, w_nk, sa, sw_gn, bias, y_f16, (int)M, (int)N, (int)K};
  float* part = pg_splitk_part(g, ws, ws_bytes, group_size);
  if (part)
    return hip_status(cider::launch_gemm_pg_splitk(g, group_size, false, cider::W_I8,
                                                   cider::pg_splitk_ways((int)M, (int)N, (int)K,
                                                                         group_size),
                                                   part, s),
                      fn);
  return hip_status(cider::launch_gemm(g, cider::W_I8, cider::EPI_PG, false, group_size, s), fn);
}

int cider_w4_repack_ref(const uint8_t* src_kn, uint8_t* dst_nk, int64_t N, int64_t K,
                        void* stream) {
  static const char* fn = "cider_w4_repack_ref";
  CIDER_TRY(check_dims(fn, 1, N, K));
  if (K % 2 != 0)
    return fail(CIDER_E_INVALID, "%s: K=%lld must be even", fn, (long long)K);
  if (N == 0 || K == 0) return ok();
  CIDER_TRY(need(fn, src_kn, "src", true));
  CIDER_TRY(need(fn, dst_nk, "dst", true));
  return hip_status(cider::launch_w4_repack_ref(src_kn, dst_nk, (int)N, (int)K,
                                                (hipStream_t)stream),
                    fn);
}

int cider_w4a8_linear(const void* x_f16, const uint8_t* w4_nk, const float* sw, void* y_f16,
                      void* ws, size_t ws_bytes, int64_t M, int64_t N, int64_t K,
                      void* stream) {
  static const char* fn = "cider_w4a8_linear";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (K % 2 != 0)
    return fail(CIDER_E_INVALID, "%s: K=%lld must be even", fn, (long long)K);
  if (M == 0 || N == 0) return ok();
  CIDER_TRY(need(fn, x_f16, "x", K > 0));
  CIDER_TRY(need(fn, w4_nk, "packed_w", K > 0));
  CIDER_TRY(need(fn, sw, "scale_w", true));
  CIDER_TRY(need(fn, y_f16, "y", true));
  const hipStream_t s = (hipStream_t)stream;
  CIDER_TRY(check_ws(fn, ws, ws_bytes, quant_ws_bytes(M, K)));
  int rc;
  const cider::GemmArgs gf{nullptr, w4_nk, nullptr, sw, nullptr, y_f16, (int)M, (int)N, (int)K};
  if (try_fused_gemv(fn, x_f16, gf, cider::W_I4, cider::EPI_PC, 0, s, &rc)) return rc;
  int8_t* q;
  float* sa;
  CIDER_TRY(quantize_into_ws(fn, x_f16, ws, M, K, s, &q, &sa));
  cider::GemmArgs g{q, w4_nk, sa, sw, nullptr, y_f16, (int)M, (int)N, (int)K};
  return hip_status(cider::launch_gemm(g, cider::W_I4, cider::EPI_PC, false, 0, s), fn);
}

int cider_w4a8_linear_ref(const void* x_f16, const uint8_t* packed_kn, const float* sw,
                          void* y_f16, void* ws, size_t ws_bytes, int64_t M, int64_t N,
                          int64_t K, void* stream) {
  static const char* fn = "cider_w4a8_linear_ref";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (K % 2 != 0)
    return fail(CIDER_E_INVALID, "%s: K=%lld must be even", fn, (long long)K);
  if (M == 0 || N == 0) return ok();
  CIDER_TRY(need(fn, x_f16, "x", K > 0));
  CIDER_TRY(need(fn, packed_kn, "packed_w", K > 0));
  CIDER_TRY(need(fn, sw, "scale_w", true));
  CIDER_TRY(need(fn, y_f16, "y", true));
  const size_t qbytes = quant_ws_bytes(M, K);
  CIDER_TRY(check_ws(fn, ws, ws_bytes, qbytes + align256((size_t)N * (size_t)(K / 2))));
  const hipStream_t s = (hipStream_t)stream;
  // The library-layout copy of the weights lives after the quantization
  // scratch; the repack is enqueued ahead of the GEMM on the same stream.
  uint8_t* w4_nk = reinterpret_cast<uint8_t*>(ws) + qbytes;
  if (K > 0)
    CIDER_TRY(hip_status(cider::launch_w4_repack_ref(packed_kn, w4_nk, (int)N, (int)K, s), fn));
  return cider_w4a8_linear(x_f16, w4_nk, sw, y_f16, ws, qbytes, M, N, K, stream);
}

int cider_w4a8_pergroup_linear(const void* x_f16, const uint8_t* w4_nk,
                               const void* scale_gn_f16, const void* bias_f16, void* y_f16,
                               void* ws, size_t ws_bytes, int64_t M, int64_t N, int64_t K,
                               int group_size, void* stream) {
  static const char* fn = "cider_w4a8_pergroup_linear";
  CIDER_TRY(check_dims(fn, M, N, K));
  if (group_size != 64 && group_size != 128)
    return fail(CIDER_E_INVALID, "%s: group_size must be 64 or 128 (got %d)", fn, group_size);
  if (K % group_size != 0)
    return fail(CIDER_E_INVALID, "%s: K=%lld is not a multiple of group_size=%d", fn,
                (long long)K, group_size);
  if (M == 0 || N == 0) return ok();
  CIDER_TRY(need(fn, x_f16, "x", K > 0));
  CIDER_TRY(need(fn, w4_nk, "packed_w", K > 0));
  CIDER_TRY(need(fn, scale_gn_f16, "scales", K > 0));
  CIDER_TRY(need(fn, y_f16, "y", true));
  const hipStream_t s = (hipStream_t)stream;
  CIDER_TRY(check_ws(fn, ws, ws_bytes, quant_ws_bytes(M, K)));
  int rc;
  const cider::GemmArgs gf{nullptr, w4_nk, nullptr, scale_gn_f16,
                           reinterpret_cast<const uint16_t*>(bias_f16), y_f16, (int)M, (int)N,
                           (int)K};
  if (try_fused_gemv(fn, x_f16, gf, cider::W_I4, cider::EPI_PG, group_size, s, &rc)) return rc;
  int8_t* q;
  float* sa;
  CIDER_TRY(quantize_into_ws(fn, x_f16, ws, M, K, s, &q, &sa));
  cider::GemmArgs g{q, w4_nk, sa, scale_gn_f16, reinterpret_cast<const uint16_t*>(bias_f16),
                    y_f16, (int)M, (int)N, (int)K};
  float* part = pg_splitk_part(g, ws, ws_bytes, group_size);
  if (part)
    return hip_status(cider::launch_gemm_pg_splitk(g, group_size, true, cider::W_I4,
                                                   cider::pg_splitk_ways((int)M, (int)N, (int)K,
                                                                         group_size),
                                                   part, s),
                      fn);
  return hip_status(cider::launch_gemm(g, cider::W_I4, cider::EPI_PG, true, group_size, s), fn);
}

// ---- producers of the linear's input and the decode attention -------------

namespace {

int check_rows(const char* fn, int64_t M, int64_t K, const char* kname) {
  CIDER_TRY(check_dims(fn, M, 1, K));
  if (K % 8 != 0)
    return fail(CIDER_E_INVALID, "%s: %s=%lld must be a multiple of 8", fn, kname, (long long)K);
  return CIDER_OK;
}

}  // namespace

int cider_rmsnorm_quantize(const void* x_f16, const void* add_f16, void* sum_f16,
                           const void* w_f16, float eps, void* y_f16, int8_t* q, float* sa,
                           int64_t M, int64_t K, void* stream) {
  static const char* fn = "cider_rmsnorm_quantize";
  CIDER_TRY(check_rows(fn, M, K, "K"));
  if (!(eps >= 0.0f)) return fail(CIDER_E_INVALID, "%s: eps must be >= 0", fn);
  if (y_f16 == nullptr && q == nullptr)
    return fail(CIDER_E_INVALID, "%s: neither y nor q requested", fn);
  if (add_f16 != nullptr && sum_f16 == nullptr)
    return fail(CIDER_E_INVALID, "%s: add given without sum", fn);
  if (M == 0 || K == 0) return ok();
  CIDER_TRY(need(fn, x_f16, "x", true));
  CIDER_TRY(need(fn, w_f16, "w", true));
  CIDER_TRY(need(fn, sa, "sa", q != nullptr));
  if (!aligned16(x_f16) || !aligned16(add_f16) || !aligned16(sum_f16) || !aligned16(w_f16) ||
      !aligned16(y_f16) || ((uintptr_t)q & 7) != 0)
    return fail(CIDER_E_INVALID, "%s: fp16 arrays must be 16-byte and q 8-byte aligned", fn);
  if (y_f16 != nullptr && (y_f16 == x_f16 || y_f16 == sum_f16))
    return fail(CIDER_E_INVALID, "%s: y must not alias x or sum", fn);
  return hip_status(
      cider::launch_rmsnorm(reinterpret_cast<const uint16_t*>(x_f16),
                            reinterpret_cast<const uint16_t*>(add_f16),
                            reinterpret_cast<uint16_t*>(sum_f16),
                            reinterpret_cast<const uint16_t*>(w_f16), eps,
                            reinterpret_cast<uint16_t*>(y_f16), q, sa, (int)M, (int)K,
                            (hipStream_t)stream),
      fn);
}

namespace {

// byte ranges [a, a + na) and [b, b + nb) overlap (either pointer NULL: no)
bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  if (a == nullptr || b == nullptr) return false;
  const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
  return pa < pb + nb && pb < pa + na;
}

int check_producer_mv(const char* fn, const void* x, const int8_t* w, const float* scale_w,
                      const void* y, int64_t N, int64_t K) {
  CIDER_TRY(check_dims(fn, 1, N, K));
  if (N < 1 || K < 1) return fail(CIDER_E_INVALID, "%s: N and K must be >= 1", fn);
  CIDER_TRY(need(fn, x, "x", true));
  CIDER_TRY(need(fn, w, "w", true));
  CIDER_TRY(need(fn, scale_w, "scale_w", true));
  CIDER_TRY(need(fn, y, "y", true));
  if (!cider::mv_producer_supported(x, w, (int)K))
    return fail(CIDER_E_UNSUPPORTED,
                "%s: needs K %% 256 == 0, K <= 16384 and 16-byte aligned x and w (K=%lld)", fn,
                (long long)K);
  if (((uintptr_t)y & 1) != 0) return fail(CIDER_E_INVALID, "%s: y must be 2-byte aligned", fn);
  return CIDER_OK;
}

}  // namespace

int cider_rmsnorm_mv(const void* x_f16, const void* add_f16, void* sum_f16, const void* norm_w_f16,
                     float eps, const int8_t* w, const float* scale_w, const void* bias_f16,
                     void* y_f16, int64_t N, int64_t K, void* stream) {
  static const char* fn = "cider_rmsnorm_mv";
  CIDER_TRY(check_producer_mv(fn, x_f16, w, scale_w, y_f16, N, K));
  if (!(eps >= 0.0f)) return fail(CIDER_E_INVALID, "%s: eps must be >= 0", fn);
  CIDER_TRY(need(fn, norm_w_f16, "norm_w", true));
  if ((add_f16 == nullptr) != (sum_f16 == nullptr))
    return fail(CIDER_E_INVALID, "%s: add and sum come together", fn);
  if (!aligned16(add_f16) || !aligned16(sum_f16) || !aligned16(norm_w_f16) ||
      ((uintptr_t)bias_f16 & 1) != 0)
    return fail(CIDER_E_INVALID, "%s: add, sum and norm_w must be 16-byte aligned", fn);
  const size_t row = (size_t)K * 2;
  if (overlaps(sum_f16, row, x_f16, row) || overlaps(sum_f16, row, add_f16, row))
    return fail(CIDER_E_INVALID, "%s: sum must not overlap x or add (other workgroups read them)",
                fn);
  if (overlaps(y_f16, (size_t)N * 2, x_f16, row) || overlaps(y_f16, (size_t)N * 2, add_f16, row) ||
      overlaps(y_f16, (size_t)N * 2, sum_f16, row))
    return fail(CIDER_E_INVALID, "%s: y must not overlap x, add or sum", fn);
  return hip_status(
      cider::launch_mv_producer(
          add_f16 ? cider::XM_ADDNORM : cider::XM_NORM, reinterpret_cast<const uint16_t*>(x_f16),
          reinterpret_cast<const uint16_t*>(add_f16), reinterpret_cast<uint16_t*>(sum_f16),
          reinterpret_cast<const uint16_t*>(norm_w_f16), eps, w, scale_w,
          reinterpret_cast<const uint16_t*>(bias_f16), reinterpret_cast<uint16_t*>(y_f16), (int)N,
          (int)K, (hipStream_t)stream),
      fn);
}

int cider_swiglu_mv(const void* gate_up_f16, const int8_t* w, const float* scale_w,
                    const void* bias_f16, void* y_f16, int64_t N, int64_t K, void* stream) {
  static const char* fn = "cider_swiglu_mv";
  CIDER_TRY(check_producer_mv(fn, gate_up_f16, w, scale_w, y_f16, N, K));
  if (((uintptr_t)bias_f16 & 1) != 0)
    return fail(CIDER_E_INVALID, "%s: bias must be 2-byte aligned", fn);
  if (overlaps(y_f16, (size_t)N * 2, gate_up_f16, (size_t)K * 4))
    return fail(CIDER_E_INVALID, "%s: y must not overlap gate_up", fn);
  return hip_status(
      cider::launch_mv_producer(cider::XM_SWIGLU, reinterpret_cast<const uint16_t*>(gate_up_f16),
                                nullptr, nullptr, nullptr, 0.0f, w, scale_w,
                                reinterpret_cast<const uint16_t*>(bias_f16),
                                reinterpret_cast<uint16_t*>(y_f16), (int)N, (int)K,
                                (hipStream_t)stream),
      fn);
}

int cider_silu_mul_quantize(const void* gu_f16, void* y_f16, int8_t* q, float* sa, int64_t M,
                            int64_t I, void* stream) {
  static const char* fn = "cider_silu_mul_quantize";
  CIDER_TRY(check_rows(fn, M, I, "I"));
  if (2 * I > kMaxDim) return fail(CIDER_E_INVALID, "%s: I above 2^29", fn);
  if (y_f16 == nullptr && q == nullptr)
    return fail(CIDER_E_INVALID, "%s: neither y nor q requested", fn);
  if (M == 0 || I == 0) return ok();
  CIDER_TRY(need(fn, gu_f16, "gate_up", true));
  CIDER_TRY(need(fn, sa, "sa", q != nullptr));
  if (!aligned16(gu_f16) || !aligned16(y_f16) || ((uintptr_t)q & 7) != 0)
    return fail(CIDER_E_INVALID, "%s: fp16 arrays must be 16-byte and q 8-byte aligned", fn);
  return hip_status(cider::launch_silu_mul(reinterpret_cast<const uint16_t*>(gu_f16),
                                           reinterpret_cast<uint16_t*>(y_f16), q, sa, (int)M,
                                           (int)I, (hipStream_t)stream),
                    fn);
}

int cider_qk_norm_rope(const void* qkv_f16, const void* q_norm_w_f16, const void* k_norm_w_f16,
                       float eps, const void* cos_f16, const void* sin_f16, int64_t P,
                       const int64_t* rope_row, const int64_t* slot, void* q_out_f16,
                       void* k_cache_f16, void* v_cache_f16, int64_t L, int64_t H, int64_t KV,
                       int64_t D, int64_t T, void* stream) {
  static const char* fn = "cider_qk_norm_rope";
  if (D != 128) return fail(CIDER_E_INVALID, "%s: head_dim must be 128 (got %lld)", fn, (long long)D);
  if (L < 0 || H <= 0 || KV <= 0 || T <= 0 || P <= 0 || L > kMaxDim || H + 2 * KV > 4096 ||
      T > kMaxDim || P > kMaxDim || L * (H + 2 * KV) > ((int64_t)1 << 31) - 4)
    return fail(CIDER_E_INVALID, "%s: bad sizes (L=%lld H=%lld KV=%lld T=%lld P=%lld)", fn,
                (long long)L, (long long)H, (long long)KV, (long long)T, (long long)P);
  if (!(eps >= 0.0f)) return fail(CIDER_E_INVALID, "%s: eps must be >= 0", fn);
  if (L == 0) return ok();
  CIDER_TRY(need(fn, qkv_f16, "qkv", true));
  CIDER_TRY(need(fn, q_norm_w_f16, "q_norm_w", true));
  CIDER_TRY(need(fn, k_norm_w_f16, "k_norm_w", true));
  CIDER_TRY(need(fn, cos_f16, "cos", true));
  CIDER_TRY(need(fn, sin_f16, "sin", true));
  CIDER_TRY(need(fn, rope_row, "rope_row", true));
  CIDER_TRY(need(fn, slot, "slot", true));
  CIDER_TRY(need(fn, q_out_f16, "q_out", true));
  CIDER_TRY(need(fn, k_cache_f16, "k_cache", true));
  CIDER_TRY(need(fn, v_cache_f16, "v_cache", true));
  return hip_status(
      cider::launch_qk_norm_rope(
          reinterpret_cast<const uint16_t*>(qkv_f16),
          reinterpret_cast<const uint16_t*>(q_norm_w_f16),
          reinterpret_cast<const uint16_t*>(k_norm_w_f16), eps,
          reinterpret_cast<const uint16_t*>(cos_f16), reinterpret_cast<const uint16_t*>(sin_f16),
          P, rope_row, slot, reinterpret_cast<uint16_t*>(q_out_f16),
          reinterpret_cast<uint16_t*>(k_cache_f16), reinterpret_cast<uint16_t*>(v_cache_f16),
          (int)L, (int)H, (int)KV, T, (hipStream_t)stream),
      fn);
}

size_t cider_attn_decode_workspace_bytes(int64_t H, int64_t T) {
  if (H <= 0 || T <= 0 || H > 4096 || T > kMaxDim) return 0;
  return align256(cider::attn_decode_ws_floats((int)H, T) * sizeof(float));
}

int cider_attn_decode(const void* q_f16, const void* k_cache_f16, const void* v_cache_f16,
                      const int64_t* n_valid, float scale, void* ws, size_t ws_bytes,
                      void* out_f16, int64_t H, int64_t KV, int64_t D, int64_t T, void* stream) {
  static const char* fn = "cider_attn_decode";
  if (D != 128) return fail(CIDER_E_INVALID, "%s: head_dim must be 128 (got %lld)", fn, (long long)D);
  if (H <= 0 || KV <= 0 || H > 4096 || H % KV != 0 ||
      (H / KV != 1 && H / KV != 2 && H / KV != 4 && H / KV != 8))
    return fail(CIDER_E_INVALID, "%s: H/KV must be 1, 2, 4 or 8 (H=%lld KV=%lld)", fn,
                (long long)H, (long long)KV);
  if (T <= 0 || T > kMaxDim || T % 8 != 0)
    return fail(CIDER_E_INVALID, "%s: cache capacity T=%lld must be a positive multiple of 8",
                fn, (long long)T);
  CIDER_TRY(need(fn, q_f16, "q", true));
  CIDER_TRY(need(fn, k_cache_f16, "k_cache", true));
  CIDER_TRY(need(fn, v_cache_f16, "v_cache", true));
  CIDER_TRY(need(fn, n_valid, "n_valid", true));
  CIDER_TRY(need(fn, out_f16, "out", true));
  CIDER_TRY(check_ws(fn, ws, ws_bytes, cider_attn_decode_workspace_bytes(H, T)));
  if (!aligned16(q_f16) || !aligned16(k_cache_f16) || !aligned16(v_cache_f16))
    return fail(CIDER_E_INVALID, "%s: q and the caches must be 16-byte aligned", fn);
  return hip_status(
      cider::launch_attn_decode(reinterpret_cast<const uint16_t*>(q_f16),
                                reinterpret_cast<const uint16_t*>(k_cache_f16),
                                reinterpret_cast<const uint16_t*>(v_cache_f16), n_valid, scale,
                                reinterpret_cast<float*>(ws), reinterpret_cast<uint16_t*>(out_f16),
                                (int)H, (int)KV, T, (hipStream_t)stream),
      fn);
}

size_t cider_attn_prefill_workspace_bytes(int64_t c, int64_t n, int64_t H) {
  if (H <= 0 || H > 4096 || c < 1 || n < c || n > ((int64_t)1 << 24) || c * H > kMaxDim)
    return 0;
  const size_t f = cider::attn_prefill_ws_floats((int)c, (int)n, (int)H);
  return f ? align256(f * sizeof(float)) : 0;
}

int cider_attn_prefill(const void* q_f16, const void* k_cache_f16, const void* v_cache_f16,
                       float scale, void* ws, size_t ws_bytes, void* out_f16, int64_t c,
                       int64_t n, const int64_t* n_dev, int64_t H, int64_t KV, int64_t D,
                       int64_t T, void* stream) {
  static const char* fn = "cider_attn_prefill";
  if (D != 128) return fail(CIDER_E_INVALID, "%s: head_dim must be 128 (got %lld)", fn, (long long)D);
  if (H <= 0 || KV <= 0 || H > 4096 || H % KV != 0)
    return fail(CIDER_E_INVALID, "%s: H=%lld must be a positive multiple of KV=%lld (H <= 4096)",
                fn, (long long)H, (long long)KV);
  if (T <= 0 || T > ((int64_t)1 << 24) || n < 1 || n > T || c < 1 || c > n || c * H > kMaxDim)
    return fail(CIDER_E_INVALID, "%s: need 1 <= c <= n <= T <= 2^24 (c=%lld n=%lld T=%lld)", fn,
                (long long)c, (long long)n, (long long)T);
  CIDER_TRY(need(fn, q_f16, "q", true));
  CIDER_TRY(need(fn, k_cache_f16, "k_cache", true));
  CIDER_TRY(need(fn, v_cache_f16, "v_cache", true));
  CIDER_TRY(need(fn, out_f16, "out", true));
  if (!aligned16(q_f16) || !aligned16(k_cache_f16) || !aligned16(v_cache_f16) ||
      !aligned16(out_f16))
    return fail(CIDER_E_INVALID, "%s: q, the caches and out must be 16-byte aligned", fn);
  if (ws != nullptr && ((uintptr_t)ws & 255) != 0)
    return fail(CIDER_E_INVALID, "%s: ws must be 256-byte aligned", fn);
  return hip_status(
      cider::launch_attn_prefill(reinterpret_cast<const uint16_t*>(q_f16),
                                 reinterpret_cast<const uint16_t*>(k_cache_f16),
                                 reinterpret_cast<const uint16_t*>(v_cache_f16),
                                 reinterpret_cast<uint16_t*>(out_f16), scale,
                                 reinterpret_cast<float*>(ws), ws ? ws_bytes / sizeof(float) : 0,
                                 (int)c, (int)n, n_dev, (int)H, (int)KV, T, (hipStream_t)stream),
      fn);
}

size_t cider_attn_prefill_quantize_workspace_bytes(int64_t c, int64_t n, int64_t H) {
  if (H <= 0 || H > 128 || c < 1 || n < c || n > ((int64_t)1 << 24) || c * H > kMaxDim) return 0;
  return align256(cider::attn_prefill_quant_ws_bytes((int)c, (int)n, (int)H));
}

int cider_attn_prefill_quantize(const void* q_f16, const void* k_cache_f16,
                                const void* v_cache_f16, float scale, void* ws, size_t ws_bytes,
                                int8_t* q_out, float* sa_out, int64_t c, int64_t n,
                                const int64_t* n_dev, int64_t H, int64_t KV, int64_t D, int64_t T,
                                void* stream) {
  static const char* fn = "cider_attn_prefill_quantize";
  if (D != 128) return fail(CIDER_E_INVALID, "%s: head_dim must be 128 (got %lld)", fn, (long long)D);
  if (H <= 0 || KV <= 0 || H > 128 || H % KV != 0)
    return fail(CIDER_E_INVALID, "%s: H=%lld must be a positive multiple of KV=%lld (H <= 128)",
                fn, (long long)H, (long long)KV);
  if (T <= 0 || T > ((int64_t)1 << 24) || n < 1 || n > T || c < 1 || c > n || c * H > kMaxDim)
    return fail(CIDER_E_INVALID, "%s: need 1 <= c <= n <= T <= 2^24 (c=%lld n=%lld T=%lld)", fn,
                (long long)c, (long long)n, (long long)T);
  CIDER_TRY(need(fn, q_f16, "q", true));
  CIDER_TRY(need(fn, k_cache_f16, "k_cache", true));
  CIDER_TRY(need(fn, v_cache_f16, "v_cache", true));
  CIDER_TRY(need(fn, q_out, "q_out", true));
  CIDER_TRY(need(fn, sa_out, "sa_out", true));
  CIDER_TRY(need(fn, ws, "ws", true));
  if (!aligned16(q_f16) || !aligned16(k_cache_f16) || !aligned16(v_cache_f16) || !aligned16(q_out))
    return fail(CIDER_E_INVALID, "%s: q, the caches and q_out must be 16-byte aligned", fn);
  if (((uintptr_t)ws & 255) != 0)
    return fail(CIDER_E_INVALID, "%s: ws must be 256-byte aligned", fn);
  const size_t need_bytes = (size_t)c * H * D * 2;
  if (ws_bytes < need_bytes)
    return fail(CIDER_E_INVALID, "%s: ws holds %zu bytes, needs at least %zu (c * H * 256)", fn,
                ws_bytes, need_bytes);
  return hip_status(
      cider::launch_attn_prefill_quant(reinterpret_cast<const uint16_t*>(q_f16),
                                       reinterpret_cast<const uint16_t*>(k_cache_f16),
                                       reinterpret_cast<const uint16_t*>(v_cache_f16), q_out,
                                       sa_out, scale, ws, ws_bytes, (int)c, (int)n, n_dev, (int)H,
                                       (int)KV, T, (hipStream_t)stream),
      fn);
}

}  // extern "C"
