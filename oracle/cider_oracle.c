/*
 * C restatement of the cider CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (as a checker of the numpy
 * oracle and of the HIP kernels) and by the cpu_baseline leg of bench.py.
 * Nothing in the product library links or calls it.
 *
 * The arithmetic is that of oracle/cider_oracle.py, which cites the
 * reference kernels line by line; this file repeats only the citations of
 * the functions it restates.  Compile without -ffast-math and with
 * -ffp-contract=off so every binary32 operation rounds on its own.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- binary16 <-> binary32 (IEEE 754, round to nearest even) ---------- */

static float h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else { /* subnormal: value = m * 2^-24, exact in binary32 */
      float v = (float)m * 5.9604644775390625e-8f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static uint16_t f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf or NaN (quiet the NaN) */
    return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
  if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
    return sign | 0x7c00u;
  if (ax < 0x38800000u) { /* below 2^-14: binary16 subnormal or zero */
    /* value / 2^-24 rounded to an integer, ties to even */
    float a;
    memcpy(&a, &ax, 4);
    float t = a * 16777216.0f; /* exact: scaling by 2^24 */
    float r = nearbyintf(t);   /* default rounding mode is RNE */
    return sign | (uint16_t)r;
  }
  /* normal: keep 10 mantissa bits, round the 13 dropped bits to even */
  uint32_t mant = ax & 0x7fffffu;
  uint32_t exp = (ax >> 23) - 112u;
  uint32_t hbits = (exp << 10) | (mant >> 13);
  uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (hbits & 1u))) hbits += 1u;
  return sign | (uint16_t)hbits;
}

void oracle_h2f_array(const uint16_t* h, float* f, int64_t n) {
  for (int64_t i = 0; i < n; i++) f[i] = h2f(h[i]);
}
void oracle_f2h_array(const float* f, uint16_t* h, int64_t n) {
  for (int64_t i = 0; i < n; i++) h[i] = f2h(f[i]);
}

/* ---- a1: per-token quantization (w8a8_quantize.metal:33-86) ---------- */

void oracle_quantize_per_token(const uint16_t* x, int M, int K, int8_t* q,
                               float* sa) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++) {
    const uint16_t* row = x + (int64_t)m * K;
    float amax = 0.0f;
    for (int k = 0; k < K; k++) amax = fmaxf(amax, fabsf(h2f(row[k])));
    float s = amax / 127.0f;
    if (s == 0.0f) s = 1.0f;
    float inv = 1.0f / s;
    sa[m] = s;
    int8_t* out = q + (int64_t)m * K;
    for (int k = 0; k < K; k++) {
      float v = h2f(row[k]) * inv;
      float r = roundf(v); /* half away from zero */
      r = fminf(fmaxf(r, -128.0f), 127.0f);
      out[k] = (int8_t)(int)r;
    }
  }
}

/* ---- a3: C = A * B^T in int32 (w8a8_matmul.metal:301-453) -------------- */

/* Integer sums are exact in any order, so the GEMM is blocked for the host:
 * 4 rows of a x 2 rows of b per register block, 16 k per step (int8 widened
 * to int16, pairwise products summed into int32 lanes by vpmaddwd), with a
 * scalar tail for K % 16.  Compiled for AVX2 and, where the host has it,
 * AVX-512BW (the same code, chosen at load time by target_clones). */
#if defined(__x86_64__) && defined(__GNUC__)
#include <immintrin.h>
#define ORACLE_X86 1
#endif

static int32_t dot_scalar(const int8_t* a, const int8_t* b, int k0, int K) {
  int32_t acc = 0;
  for (int k = k0; k < K; k++) acc += (int32_t)a[k] * (int32_t)b[k];
  return acc;
}

#ifdef ORACLE_X86
__attribute__((target("avx2"))) static inline int32_t hsum8(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
  return _mm_cvtsi128_si32(s);
}

/* c[i][j] = sum_k a_i[k] b_j[k] for i < 4, j < 2 */
__attribute__((target("avx2"))) static void block4x2(const int8_t* a0, int64_t lda,
                                                     const int8_t* b0, int64_t ldb, int K,
                                                     int32_t c[4][2]) {
  __m256i acc[4][2];
  for (int i = 0; i < 4; i++) acc[i][0] = acc[i][1] = _mm256_setzero_si256();
  const int K16 = K & ~15;
  for (int k = 0; k < K16; k += 16) {
    __m256i bv0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(b0 + k)));
    __m256i bv1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(b0 + ldb + k)));
    for (int i = 0; i < 4; i++) {
      __m256i av = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(a0 + i * lda + k)));
      acc[i][0] = _mm256_add_epi32(acc[i][0], _mm256_madd_epi16(av, bv0));
      acc[i][1] = _mm256_add_epi32(acc[i][1], _mm256_madd_epi16(av, bv1));
    }
  }
  for (int i = 0; i < 4; i++)
    for (int j = 0; j < 2; j++)
      c[i][j] = hsum8(acc[i][j]) + dot_scalar(a0 + i * lda, b0 + j * ldb, K16, K);
}

static int have_avx2(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2");
}
#endif

void oracle_i8_gemm_nt(const int8_t* a, const int8_t* b, int M, int N, int K,
                       int32_t* c) {
  const int NB = 64;
#ifdef ORACLE_X86
  const int simd = have_avx2();
#else
  const int simd = 0;
#endif
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int m0 = 0; m0 < M; m0 += 4) {
    for (int n0 = 0; n0 < N; n0 += NB) {
      int m1 = m0 + 4 < M ? m0 + 4 : M;
      int n1 = n0 + NB < N ? n0 + NB : N;
      int n = n0;
#ifdef ORACLE_X86
      if (simd && m1 - m0 == 4) {
        for (; n + 2 <= n1; n += 2) {
          int32_t blk[4][2];
          block4x2(a + (int64_t)m0 * K, K, b + (int64_t)n * K, K, K, blk);
          for (int i = 0; i < 4; i++) {
            c[(int64_t)(m0 + i) * N + n] = blk[i][0];
            c[(int64_t)(m0 + i) * N + n + 1] = blk[i][1];
          }
        }
      }
#endif
      for (int m = m0; m < m1; m++)
        for (int nn = n; nn < n1; nn++)
          c[(int64_t)m * N + nn] = dot_scalar(a + (int64_t)m * K, b + (int64_t)nn * K, 0, K);
    }
  }
}

/* ---- a2: per-channel epilogue (w8a8_matmul.metal:74-77) ---------------- */

void oracle_dequant_perchannel(const int32_t* acc, const float* sa,
                               const float* sw, const uint16_t* bias, int M,
                               int N, uint16_t* y) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++) {
    for (int n = 0; n < N; n++) {
      float v = (float)acc[(int64_t)m * N + n];
      v = v * sa[m];
      v = v * sw[n];
      if (bias) v = v + h2f(bias[n]);
      y[(int64_t)m * N + n] = f2h(v);
    }
  }
}

/* ---- a4: M == 1 per-channel MV (w8a8_int8_mv.metal:26-70) -------------- */

void oracle_mv_perchannel(const uint16_t* x, const int8_t* w, const float* sw,
                          const uint16_t* bias, int N, int K, uint16_t* y) {
  int nb = (K + 255) / 256;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    float r[32];
    for (int l = 0; l < 32; l++) r[l] = 0.0f;
    for (int b = 0; b < nb; b++) {
      for (int l = 0; l < 32; l++) {
        float d = 0.0f;
        for (int i = 0; i < 8; i++) {
          int k = 256 * b + 8 * l + i;
          float p = k < K ? (float)w[(int64_t)n * K + k] * h2f(x[k]) : 0.0f;
          d = i == 0 ? p : d + p;
        }
        r[l] = r[l] + d;
      }
    }
    for (int off = 16; off >= 1; off >>= 1) {
      float t[32];
      for (int l = 0; l < 32; l++) t[l] = r[l] + r[l ^ off];
      for (int l = 0; l < 32; l++) r[l] = t[l];
    }
    float v = sw[n] * r[0];
    v = v + h2f(bias[n]);
    y[n] = f2h(v);
  }
}

/* ---- a5: per-group GEMM (pergroup_int8_gemm.metal:90-191) -------------- */

void oracle_pergroup_gemm(const int8_t* q, const float* sa, const int8_t* w,
                          const float* sw_gn, const uint16_t* bias, int M,
                          int N, int K, int gs, uint16_t* y) {
  int G = K / gs;
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; m++) {
    const int8_t* ar = q + (int64_t)m * K;
    for (int n = 0; n < N; n++) {
      const int8_t* br = w + (int64_t)n * K;
      float acc = 0.0f;
      for (int g = 0; g < G; g++) {
        int32_t d = 0;
        for (int k = g * gs; k < (g + 1) * gs; k++)
          d += (int32_t)ar[k] * (int32_t)br[k];
        float t = (float)d * sw_gn[(int64_t)g * N + n];
        acc = acc + t;
      }
      float v = acc * sa[m];
      if (bias) v = v + h2f(bias[n]);
      y[(int64_t)m * N + n] = f2h(v);
    }
  }
}

/* ---- full per-channel linear, M >= 2 (w8a8_primitive.mm:179-251) ------- */

void oracle_perchannel_linear(const uint16_t* x, const int8_t* w,
                              const float* sw, const uint16_t* bias, int M,
                              int N, int K, int8_t* q_ws, float* sa_ws,
                              int32_t* acc_ws, uint16_t* y) {
  oracle_quantize_per_token(x, M, K, q_ws, sa_ws);
  oracle_i8_gemm_nt(q_ws, w, M, N, K, acc_ws);
  oracle_dequant_perchannel(acc_ws, sa_ws, sw, bias, M, N, y);
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
