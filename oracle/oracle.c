/*
 * CPU oracle for the xpu_playground decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker / CPU baseline; the product
 * library never links or loads it. The order conventions are described in
 * oracle.h. Citations are reference file:line (xpu_playground repository).
 *
 * Build: see oracle/Makefile (gcc -O3 -mfma -ffp-contract=off -fopenmp).
 * -ffp-contract=off keeps every a*b+c that is not written as fmaf() as two
 * roundings; -mfma makes fmaf() a single hardware instruction.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;
void orc_set_threads(int n) { g_threads = n; }
int orc_get_threads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ codecs */

/* qwen3/model.cpp:497-502 (= level_zero/peak_l0.cpp:726-731): round to
 * nearest even by adding 0x7fff + lsb, no NaN special case. */
uint16_t orc_f32_to_bf16(float v) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

/* qwen3/model.cpp:503-508 */
float orc_bf16_to_f32(uint16_t v) {
  uint32_t bits = (uint32_t)v << 16;
  float r;
  memcpy(&r, &bits, 4);
  return r;
}

/* level_zero/peak_l0.cpp:740-761: RNE with subnormals (shift then round),
 * overflow and NaN to Inf. */
uint16_t orc_f32_to_fp16(float v) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  int exponent = (int)((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mantissa = bits & 0x7fffffu;
  if (exponent <= 0) {
    if (exponent < -10) return (uint16_t)sign;
    mantissa = (mantissa | 0x800000u) >> (1 - exponent);
    return (uint16_t)(sign | ((mantissa + 0xfffu + ((mantissa >> 13) & 1u)) >> 13));
  }
  if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  mantissa += 0xfffu + ((mantissa >> 13) & 1u);
  if (mantissa & 0x800000u) {
    mantissa = 0;
    if (++exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  }
  return (uint16_t)(sign | ((uint32_t)exponent << 10) | (mantissa >> 13));
}

/* level_zero/peak_l0.cpp:763-785 */
float orc_fp16_to_f32(uint16_t v) {
  const uint32_t sign = (uint32_t)(v & 0x8000u) << 16;
  uint32_t exponent = (v >> 10) & 0x1fu;
  uint32_t mantissa = v & 0x3ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      int shift = 0;
      while ((mantissa & 0x400u) == 0) { mantissa <<= 1; ++shift; }
      mantissa &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 14 - shift) << 23) | (mantissa << 13);
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  float r;
  memcpy(&r, &bits, 4);
  return r;
}

/* level_zero/peak_l0.cpp:787-793 */
uint16_t orc_encode(float v, int dtype) { return dtype ? orc_f32_to_fp16(v) : orc_f32_to_bf16(v); }
float orc_decode(uint16_t v, int dtype) { return dtype ? orc_fp16_to_f32(v) : orc_bf16_to_f32(v); }

void orc_encode_n(const float *in, uint16_t *out, size_t n, int dtype) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_encode(in[i], dtype);
}
void orc_decode_n(const uint16_t *in, float *out, size_t n, int dtype) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_decode(in[i], dtype);
}

/* ------------------------------------------------------------------ synth */

/* splitmix64 finaliser (Steele, Lea, Flood, "Fast splittable pseudorandom
 * number generators", OOPSLA 2014); counter-based so any element can be
 * generated independently. */
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t orc_hash(uint64_t seed, uint64_t index) {
  return mix64(mix64(seed) + (index + 1) * 0x9e3779b97f4a7c15ull);
}

static inline float uniform_pm1(uint64_t h) {
  /* 24-bit uniform u, value (2u - 2^24) / 2^24 in [-1, 1): exact in FP32 */
  const int32_t u = (int32_t)(h >> 40);
  return (float)(2 * u - (1 << 24)) * 0x1p-24f;
}

void orc_fill_uniform(uint16_t *out, uint64_t n, uint64_t seed, int dtype) {
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
  for (int64_t i = 0; i < (int64_t)n; ++i)
    out[i] = orc_encode(uniform_pm1(orc_hash(seed, (uint64_t)i)), dtype);
}

static inline double normal_from_hash(uint64_t h) {
  const double u1 = (double)((h >> 40) + 1) * 0x1p-24;        /* (0, 1] */
  const double u2 = (double)((h >> 16) & 0xffffffu) * 0x1p-24; /* [0, 1) */
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_fill_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed, float stddev) {
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
  for (int64_t i = 0; i < (int64_t)n; ++i)
    out[i] = orc_f32_to_bf16((float)(normal_from_hash(orc_hash(seed, (uint64_t)i)) * stddev));
}

void orc_fill_gain_bf16(uint16_t *out, uint64_t n, uint64_t seed, float stddev) {
  for (uint64_t i = 0; i < n; ++i)
    out[i] = orc_f32_to_bf16(
        stddev == 0.0f ? 1.0f : (float)(1.0 + normal_from_hash(orc_hash(seed, i)) * stddev));
}

void orc_fill_tokens(uint32_t *out, uint64_t n, uint64_t seed, uint32_t vocab) {
  for (uint64_t i = 0; i < n; ++i)
    out[i] = (uint32_t)(((orc_hash(seed, i) >> 32) * (uint64_t)vocab) >> 32);
}

/* gemv.cpp:91-103 (level_zero/peak_l0.cpp:825-836): hash of the linear index
 * of the (padded, leading dimension ld) matrix and of the vector index. */
void orc_fill_reference_gemv(uint16_t *matrix, uint16_t *vector, uint32_t m,
                             uint32_t k, uint32_t ld, int dtype) {
  for (uint64_t r = 0; r < m; ++r)
    for (uint64_t c = 0; c < ld; ++c) {
      uint32_t bits = (uint32_t)(r * ld + c);
      bits ^= bits >> 16;
      bits *= 0x7feb352du;
      bits ^= bits >> 15;
      bits *= 0x846ca68bu;
      bits ^= bits >> 16;
      matrix[r * ld + c] = orc_encode(0.25f + (float)(bits & 255u) / 1024.0f, dtype);
    }
  for (uint32_t c = 0; c < k; ++c) {
    const uint32_t bits = c * 747796405u;
    vector[c] = orc_encode(0.5f + (float)((bits >> 16) & 127u) / 512.0f, dtype);
  }
}

/* ------------------------------------------------------------------ sums */

/* Canonical 64-lane x 8-slot FP32 reduction (oracle.h). acc has 512 slots:
 * lane L slot e is acc[8L + e] = acc[k & 511]. */
static float canonical_finish(const float *acc) {
  float s[64], t[64];
  for (int L = 0; L < 64; ++L) {
    const float *a = acc + 8 * L;
    s[L] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  }
  for (int m = 32; m >= 1; m >>= 1) {
    for (int L = 0; L < 64; ++L) t[L] = s[L] + s[L ^ m];
    memcpy(s, t, sizeof(s));
  }
  return s[0];
}

float orc_canonical_sum(const float *terms, uint32_t n) {
  float acc[512];
  memset(acc, 0, sizeof(acc));
  for (uint32_t k = 0; k < n; ++k) acc[k & 511] = acc[k & 511] + terms[k];
  return canonical_finish(acc);
}

/* sum of per-4096 chunk canonical sums, ascending, from +0 */
static float chunked_canonical_sum(const float *terms, uint32_t n) {
  float total = 0.0f;
  for (uint32_t c = 0; c < n; c += 4096) {
    const uint32_t len = n - c < 4096 ? n - c : 4096;
    total = total + orc_canonical_sum(terms + c, len);
  }
  return total;
}

static float canonical_dot_f(const float *a, const float *x, uint32_t k) {
  float acc[512];
  memset(acc, 0, sizeof(acc));
  uint32_t base = 0;
  for (; base + 512 <= k; base += 512)
    for (int i = 0; i < 512; ++i) acc[i] = fmaf(a[base + i], x[base + i], acc[i]);
  for (uint32_t i = 0; base + i < k; ++i) acc[i] = fmaf(a[base + i], x[base + i], acc[i]);
  return canonical_finish(acc);
}

float orc_canonical_dot(const uint16_t *a, const uint16_t *x, uint32_t k, int dtype) {
  float *af = (float *)malloc(sizeof(float) * k * 2u + 4);
  float *xf = af + k;
  orc_decode_n(a, af, k, dtype);
  orc_decode_n(x, xf, k, dtype);
  const float r = canonical_dot_f(af, xf, k);
  free(af);
  return r;
}

/* lane-local 8-slot dot used for attention scores: slot d % 8, ascending,
 * then ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7)) */
static float dot_lane8(const float *a, const float *b, uint32_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (uint32_t d = 0; d < n; ++d) acc[d & 7] = fmaf(a[d], b[d], acc[d & 7]);
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

/* ------------------------------------------------------------------ GEMV */

void orc_gemv_rows_seq(const uint16_t *a, const uint16_t *x, float *y,
                       uint32_t rows, uint32_t k, uint64_t lda, int dtype) {
  float *xf = (float *)malloc(sizeof(float) * (k ? k : 1));
  orc_decode_n(x, xf, k, dtype);
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
  for (int64_t r = 0; r < (int64_t)rows; ++r) {
    const uint16_t *row = a + (uint64_t)r * lda;
    float expected = 0.0f;
    for (uint32_t c = 0; c < k; ++c) expected += orc_decode(row[c], dtype) * xf[c];
    y[r] = expected;
  }
  free(xf);
}

void orc_gemv_f64(const uint16_t *a, const uint16_t *x, double *y, uint32_t m,
                  uint32_t k, uint64_t lda, int dtype) {
  double *xd = (double *)malloc(sizeof(double) * (k ? k : 1));
  for (uint32_t c = 0; c < k; ++c) xd[c] = orc_decode(x[c], dtype);
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
  for (int64_t r = 0; r < (int64_t)m; ++r) {
    const uint16_t *row = a + (uint64_t)r * lda;
    double s = 0.0;
    for (uint32_t c = 0; c < k; ++c) s += (double)orc_decode(row[c], dtype) * xd[c];
    y[r] = s;
  }
  free(xd);
}

void orc_gemv_canonical(const uint16_t *a, const uint16_t *x, uint16_t *y,
                        uint32_t m, uint32_t k, uint64_t lda, int dtype) {
  float *xf = (float *)malloc(sizeof(float) * (k ? k : 1));
  orc_decode_n(x, xf, k, dtype);
#pragma omp parallel num_threads(orc_get_threads())
  {
    float *row = (float *)malloc(sizeof(float) * (k ? k : 1));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < (int64_t)m; ++r) {
      orc_decode_n(a + (uint64_t)r * lda, row, k, dtype);
      y[r] = orc_encode(canonical_dot_f(row, xf, k), dtype);
    }
    free(row);
  }
  free(xf);
}

static double now_seconds(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

double orc_time_gemv_seq(const uint16_t *a, const uint16_t *x, float *y,
                         uint32_t m, uint32_t k, int dtype, int threads) {
  const int saved = g_threads;
  g_threads = threads;
  const double t0 = now_seconds();
  orc_gemv_rows_seq(a, x, y, m, k, k, dtype);
  const double t1 = now_seconds();
  g_threads = saved;
  return t1 - t0;
}

/* ------------------------------------------------------------------ GEMM */

void orc_gemm_f64(const uint16_t *a, const uint16_t *b, double *c, uint32_t m,
                  uint32_t n, uint32_t k, int dtype, const uint32_t *rows,
                  uint32_t nrows) {
  const uint32_t count = rows ? nrows : m;
  double *bd = (double *)malloc(sizeof(double) * (uint64_t)k * n + 8);
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
  for (int64_t i = 0; i < (int64_t)k * n; ++i) bd[i] = orc_decode(b[i], dtype);
  enum { RB = 16, KB = 256 };
#pragma omp parallel for schedule(dynamic, 1) num_threads(orc_get_threads())
  for (int64_t r0 = 0; r0 < (int64_t)count; r0 += RB) {
    const uint32_t rb = count - (uint32_t)r0 < RB ? count - (uint32_t)r0 : RB;
    double *acc = (double *)calloc((uint64_t)rb * n, sizeof(double));
    for (uint32_t k0 = 0; k0 < k; k0 += KB) {
      const uint32_t kend = k0 + KB < k ? k0 + KB : k;
      for (uint32_t i = 0; i < rb; ++i) {
        const uint32_t row = rows ? rows[r0 + i] : (uint32_t)(r0 + i);
        double *crow = acc + (uint64_t)i * n;
        for (uint32_t kk = k0; kk < kend; ++kk) {
          const double av = orc_decode(a[(uint64_t)row * k + kk], dtype);
          const double *brow = bd + (uint64_t)kk * n;
          for (uint32_t j = 0; j < n; ++j) crow[j] += av * brow[j];
        }
      }
    }
    memcpy(c + (uint64_t)r0 * n, acc, sizeof(double) * (uint64_t)rb * n);
    free(acc);
  }
  free(bd);
}

/* gemv.cpp:126-130 check order (the FP32 host sum, ascending k), applied to
 * each GEMM element */
void orc_gemm_f32_rows(const uint16_t *a, const uint16_t *b, float *c, uint32_t m,
                       uint32_t n, uint32_t k, int dtype, const uint32_t *rows,
                       uint32_t nrows) {
  (void)m;
  const uint32_t count = rows ? nrows : m;
  float *bf = (float *)malloc(sizeof(float) * (uint64_t)k * n + 4);
  orc_decode_n(b, bf, (uint64_t)k * n, dtype);
#pragma omp parallel for schedule(dynamic, 1) num_threads(orc_get_threads())
  for (int64_t i = 0; i < (int64_t)count; ++i) {
    const uint32_t row = rows ? rows[i] : (uint32_t)i;
    float *crow = c + (uint64_t)i * n;
    for (uint32_t j = 0; j < n; ++j) crow[j] = 0.0f;
    for (uint32_t kk = 0; kk < k; ++kk) {
      const float av = orc_decode(a[(uint64_t)row * k + kk], dtype);
      const float *brow = bf + (uint64_t)kk * n;
      for (uint32_t j = 0; j < n; ++j) crow[j] = crow[j] + av * brow[j];
    }
  }
  free(bf);
}

/* The same sums (each C element accumulates its K products in ascending k,
 * FP32, no contraction) with the loops blocked for the host caches: a
 * 64-row x 512-column C tile stays in L2 while 256-deep panels of A and B
 * stream through it. Bitwise equal to orc_gemm_f32_rows; the CPU baseline of
 * the GEMM lines (BASELINE plan: blocked FP32, all host threads). */
void orc_gemm_f32_blocked(const uint16_t *a, const uint16_t *b, float *c, uint32_t m,
                          uint32_t n, uint32_t k, int dtype) {
  enum { RB = 64, CB = 512, KB = 256 };
  float *bf = (float *)malloc(sizeof(float) * (uint64_t)k * n + 4);
  orc_decode_n(b, bf, (uint64_t)k * n, dtype);
  const int64_t row_blocks = ((int64_t)m + RB - 1) / RB, col_blocks = ((int64_t)n + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic, 1) num_threads(orc_get_threads())
  for (int64_t t = 0; t < row_blocks * col_blocks; ++t) {
    const uint32_t r0 = (uint32_t)(t / col_blocks) * RB, c0 = (uint32_t)(t % col_blocks) * CB;
    const uint32_t r1 = r0 + RB < m ? r0 + RB : m, c1 = c0 + CB < n ? c0 + CB : n;
    float arow[KB];
    for (uint32_t r = r0; r < r1; ++r)
      for (uint32_t j = c0; j < c1; ++j) c[(uint64_t)r * n + j] = 0.0f;
    for (uint32_t k0 = 0; k0 < k; k0 += KB) {
      const uint32_t k1 = k0 + KB < k ? k0 + KB : k;
      for (uint32_t r = r0; r < r1; ++r) {
        for (uint32_t kk = k0; kk < k1; ++kk) arow[kk - k0] = orc_decode(a[(uint64_t)r * k + kk], dtype);
        float *crow = c + (uint64_t)r * n;
        for (uint32_t kk = k0; kk < k1; ++kk) {
          const float av = arow[kk - k0];
          const float *brow = bf + (uint64_t)kk * n;
          for (uint32_t j = c0; j < c1; ++j) crow[j] = crow[j] + av * brow[j];
        }
      }
    }
  }
  free(bf);
}

double orc_time_gemm_blocked(const uint16_t *a, const uint16_t *b, float *c, uint32_t m,
                             uint32_t n, uint32_t k, int dtype, int threads) {
  const int saved = g_threads;
  g_threads = threads;
  const double t0 = now_seconds();
  orc_gemm_f32_blocked(a, b, c, m, n, k, dtype);
  const double t1 = now_seconds();
  g_threads = saved;
  return t1 - t0;
}

double orc_time_gemm_f32(const uint16_t *a, const uint16_t *b, float *c,
                         uint32_t m, uint32_t n, uint32_t k, int dtype,
                         uint32_t row_limit, int threads) {
  const int saved = g_threads;
  g_threads = threads;
  const uint32_t rows = row_limit && row_limit < m ? row_limit : m;
  const double t0 = now_seconds();
  orc_gemm_f32_rows(a, b, c, rows, n, k, dtype, NULL, rows);
  const double t1 = now_seconds();
  g_threads = saved;
  return t1 - t0;
}

/* ------------------------------------------------------------------ Qwen3 ops */

/* exp by Cody-Waite reduction x = n ln2 + r, |r| <= ln2/2, and the degree-7
 * Taylor polynomial of e^r in Horner form (all fmaf), scaled by 2^n. Max
 * error about 1 ulp. The gfx950 kernels evaluate the same operation sequence,
 * so both sides produce the same bits. */
static inline float pow2i(int e) {
  uint32_t bits = (uint32_t)(e + 127) << 23;
  float r;
  memcpy(&r, &bits, 4);
  return r;
}

float orc_exp(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.972084045410156f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860676533018704504e-06f, r);
  float p = 1.98412698412698412526e-04f;
  p = fmaf(p, r, 1.38888888888888894189e-03f);
  p = fmaf(p, r, 8.33333333333333321769e-03f);
  p = fmaf(p, r, 4.16666666666666643537e-02f);
  p = fmaf(p, r, 1.66666666666666657415e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int e = (int)n;
  if (e > 127) { p = p * 2.0f; e -= 1; }
  if (e < -126) return (p * pow2i(e + 64)) * 0x1p-64f;
  return p * pow2i(e);
}

static inline float bf(float v) { return orc_bf16_to_f32(orc_f32_to_bf16(v)); }

/* qwen3/kernels.hpp:36-56 (RmsNorm) with transformers Qwen3RMSNorm rounding:
 * out = bf16(w * bf16(x * (1 / sqrt(mean(x^2) + eps)))) */
void orc_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *out,
                 uint32_t width, float eps) {
  float *xf = (float *)malloc(sizeof(float) * width);
  float acc[512];
  memset(acc, 0, sizeof(acc));
  for (uint32_t k = 0; k < width; ++k) {
    xf[k] = orc_bf16_to_f32(x[k]);
    acc[k & 511] = fmaf(xf[k], xf[k], acc[k & 511]);
  }
  const float mean = canonical_finish(acc) / (float)width;
  const float scale = 1.0f / sqrtf(mean + eps);
  for (uint32_t k = 0; k < width; ++k)
    out[k] = orc_f32_to_bf16(orc_bf16_to_f32(w[k]) * bf(xf[k] * scale));
  free(xf);
}

/* qwen3/main.cpp:299-318 (upload_rope) with transformers
 * Qwen3RotaryEmbedding arithmetic: inv_freq = 1 / theta^(2i/d) in FP32,
 * angle = fp32(pos * inv_freq), cos/sin of the FP32 angle, then bf16;
 * entry d uses frequency d % (d/2). */
void orc_rope_tables(uint16_t *cos_t, uint16_t *sin_t, uint32_t max_seq,
                     uint32_t head_dim, double theta) {
  const uint32_t half = head_dim / 2;
  float *inv = (float *)malloc(sizeof(float) * half);
  for (uint32_t i = 0; i < half; ++i) {
    const float expo = (float)(2 * i) / (float)head_dim;
    inv[i] = 1.0f / (float)pow((double)(float)theta, (double)expo);
  }
  for (uint32_t p = 0; p < max_seq; ++p)
    for (uint32_t d = 0; d < head_dim; ++d) {
      const float angle = (float)p * inv[d % half];
      cos_t[(uint64_t)p * head_dim + d] = orc_f32_to_bf16((float)cos((double)angle));
      sin_t[(uint64_t)p * head_dim + d] = orc_f32_to_bf16((float)sin((double)angle));
    }
  free(inv);
}

/* qwen3/kernels.hpp:71-125 (QkvRopeCache per head) with transformers
 * rounding: RMSNorm over the head, then
 * out[i] = bf16(bf16(v[i]*cos[i]) + bf16(rotate_half(v)[i]*sin[i])). */
void orc_qk_norm_rope(uint16_t *vec, const uint16_t *norm_w, const uint16_t *cos_row,
                      const uint16_t *sin_row, uint32_t head_dim, float eps) {
  uint16_t normed[512];
  orc_rmsnorm(vec, norm_w, normed, head_dim, eps);
  const uint32_t half = head_dim / 2;
  for (uint32_t i = 0; i < head_dim; ++i) {
    const float v = orc_bf16_to_f32(normed[i]);
    const float rot = i < half ? -orc_bf16_to_f32(normed[i + half])
                               : orc_bf16_to_f32(normed[i - half]);
    const float a = bf(v * orc_bf16_to_f32(cos_row[i]));
    const float b = bf(rot * orc_bf16_to_f32(sin_row[i]));
    vec[i] = orc_f32_to_bf16(a + b);
  }
}

/* qwen3/kernels.hpp:157-192 (Attention) with transformers eager rounding:
 * s_t = bf16(bf16(q.k_t) * scale); p_t = bf16(exp(s_t - max) * (1/sum));
 * out = bf16(sum_t p_t v_t). Orders: q.k_t lane-local 8-slot; the sum of
 * exponentials chunked canonical; sum_t p_t v_t[d] in 16 residue classes
 * t % 16 (ascending t, per 4096-position chunk, chunks added ascending),
 * combined by a balanced binary tree over the residues. */
void orc_attention_head(const uint16_t *q, const uint16_t *kcache,
                        const uint16_t *vcache, uint64_t stride, uint32_t n,
                        uint32_t head_dim, uint16_t *out) {
  float qf[512], kf[512];
  for (uint32_t d = 0; d < head_dim; ++d) qf[d] = orc_bf16_to_f32(q[d]);
  const float scale = (float)(1.0 / sqrt((double)head_dim));
  float *s = (float *)malloc(sizeof(float) * (n ? n : 1) * 2);
  float *e = s + n;
  float mx = -INFINITY;
  for (uint32_t t = 0; t < n; ++t) {
    for (uint32_t d = 0; d < head_dim; ++d) kf[d] = orc_bf16_to_f32(kcache[t * stride + d]);
    s[t] = bf(bf(dot_lane8(qf, kf, head_dim)) * scale);
    if (s[t] > mx) mx = s[t];
  }
  for (uint32_t t = 0; t < n; ++t) e[t] = orc_exp(s[t] - mx);
  const float inv = 1.0f / chunked_canonical_sum(e, n);
  for (uint32_t t = 0; t < n; ++t) e[t] = bf(e[t] * inv);
  for (uint32_t d = 0; d < head_dim; ++d) {
    float res[16];
    for (int r = 0; r < 16; ++r) {
      float total = 0.0f;
      for (uint32_t c = 0; c < n; c += 4096) {
        float part = 0.0f;
        const uint32_t end = c + 4096 < n ? c + 4096 : n;
        for (uint32_t t = c + (uint32_t)r; t < end; t += 16)
          part = fmaf(e[t], orc_bf16_to_f32(vcache[t * stride + d]), part);
        total = total + part;
      }
      res[r] = total;
    }
    for (int w = 16; w > 1; w >>= 1)
      for (int r = 0; r < w / 2; ++r) res[r] = res[2 * r] + res[2 * r + 1];
    out[d] = orc_f32_to_bf16(res[0]);
  }
  free(s);
}

/* qwen3/kernels.hpp:194-207 */
void orc_add(uint16_t *left, const uint16_t *right, uint32_t width) {
  for (uint32_t i = 0; i < width; ++i)
    left[i] = orc_f32_to_bf16(orc_bf16_to_f32(left[i]) + orc_bf16_to_f32(right[i]));
}

/* qwen3/kernels.hpp:209-223 with transformers rounding:
 * gate = bf16(bf16(g / (1 + exp(-g))) * up) */
void orc_silu_mul(uint16_t *gate, const uint16_t *up, uint32_t width) {
  for (uint32_t i = 0; i < width; ++i) {
    const float g = orc_bf16_to_f32(gate[i]);
    const float act = bf(g / (1.0f + orc_exp(-g)));
    gate[i] = orc_f32_to_bf16(act * orc_bf16_to_f32(up[i]));
  }
}

/* qwen3/kernels.hpp:225-246: first maximum, NaN/Inf -> 0xffffffff */
uint32_t orc_argmax(const uint16_t *logits, uint32_t width) {
  float best = -INFINITY;
  uint32_t best_index = 0;
  for (uint32_t i = 0; i < width; ++i) {
    const float v = orc_bf16_to_f32(logits[i]);
    if (v != v || v == INFINITY || v == -INFINITY) return 0xffffffffu;
    if (v > best) { best = v; best_index = i; }
  }
  return best_index;
}

/* ------------------------------------------------------------------ Qwen3 engine */

struct orc_qwen3 {
  orc_qwen3_config c;
  uint32_t max_seq;
  uint16_t *embed, *final_norm, *lm_head;
  uint16_t **w; /* [layer * 11 + kind] for kinds 0..10 */
  uint16_t *kcache, *vcache; /* [layer][kv][max_seq][head_dim] */
  uint16_t *cos_t, *sin_t;
  uint16_t *x, *norm, *q, *k, *v, *attn, *tmp, *gate, *up, *logits;
};

uint64_t orc_qwen3_tensor_elems(const orc_qwen3_config *c, int kind) {
  const uint64_t h = c->hidden, qd = (uint64_t)c->heads * c->head_dim,
                 kvd = (uint64_t)c->kv_heads * c->head_dim, in = c->intermediate;
  switch (kind) {
  case ORC_W_Q: return qd * h;
  case ORC_W_K: case ORC_W_V: return kvd * h;
  case ORC_W_O: return h * qd;
  case ORC_W_QNORM: case ORC_W_KNORM: return c->head_dim;
  case ORC_W_GATE: case ORC_W_UP: return in * h;
  case ORC_W_DOWN: return h * in;
  case ORC_W_INNORM: case ORC_W_POSTNORM: case ORC_W_FINALNORM: return h;
  case ORC_W_EMBED: case ORC_W_LMHEAD: return (uint64_t)c->vocab * h;
  default: return 0;
  }
}

/* Synthetic weights: N(0, 0.02^2) matrices, norm gains 1 + N(0, gain_std^2)
 * (exactly 1.0 for gain_std = 0). Each tensor has its own seed stream. */
static uint64_t tensor_seed(uint64_t seed, int kind, uint32_t layer) {
  return mix64(seed ^ (0x51ed270b27e5a3c1ull * (uint64_t)(kind + 1)) ^
               (0x2545f4914f6cdd1dull * (uint64_t)(layer + 1)));
}

void orc_qwen3_fill_tensor(const orc_qwen3_config *c, uint64_t seed, float gain_std,
                           int kind, uint32_t layer, uint16_t *out) {
  const uint64_t n = orc_qwen3_tensor_elems(c, kind);
  const uint64_t ts = tensor_seed(seed, kind, layer);
  if (kind == ORC_W_QNORM || kind == ORC_W_KNORM || kind == ORC_W_INNORM ||
      kind == ORC_W_POSTNORM || kind == ORC_W_FINALNORM)
    orc_fill_gain_bf16(out, n, ts, gain_std);
  else
    orc_fill_normal_bf16(out, n, ts, 0.02f);
}

orc_qwen3 *orc_qwen3_create(const orc_qwen3_config *c, uint64_t seed,
                            float gain_std, uint32_t max_seq) {
  orc_qwen3 *m = (orc_qwen3 *)calloc(1, sizeof(orc_qwen3));
  m->c = *c;
  m->max_seq = max_seq;
  m->w = (uint16_t **)calloc((size_t)c->layers * 11, sizeof(uint16_t *));
  for (uint32_t l = 0; l < c->layers; ++l)
    for (int kind = 0; kind <= ORC_W_POSTNORM; ++kind) {
      uint16_t *t = (uint16_t *)malloc(2 * orc_qwen3_tensor_elems(c, kind));
      orc_qwen3_fill_tensor(c, seed, gain_std, kind, l, t);
      m->w[l * 11 + kind] = t;
    }
  m->embed = (uint16_t *)malloc(2 * orc_qwen3_tensor_elems(c, ORC_W_EMBED));
  orc_qwen3_fill_tensor(c, seed, gain_std, ORC_W_EMBED, 0, m->embed);
  m->final_norm = (uint16_t *)malloc(2 * (uint64_t)c->hidden);
  orc_qwen3_fill_tensor(c, seed, gain_std, ORC_W_FINALNORM, 0, m->final_norm);
  m->lm_head = m->embed;
  if (!c->tied) {
    m->lm_head = (uint16_t *)malloc(2 * orc_qwen3_tensor_elems(c, ORC_W_LMHEAD));
    orc_qwen3_fill_tensor(c, seed, gain_std, ORC_W_LMHEAD, 0, m->lm_head);
  }
  const uint64_t cache = (uint64_t)c->layers * c->kv_heads * max_seq * c->head_dim;
  m->kcache = (uint16_t *)calloc(cache, 2);
  m->vcache = (uint16_t *)calloc(cache, 2);
  m->cos_t = (uint16_t *)malloc(2 * (uint64_t)max_seq * c->head_dim);
  m->sin_t = (uint16_t *)malloc(2 * (uint64_t)max_seq * c->head_dim);
  orc_rope_tables(m->cos_t, m->sin_t, max_seq, c->head_dim, c->rope_theta);
  const uint64_t qd = (uint64_t)c->heads * c->head_dim, kvd = (uint64_t)c->kv_heads * c->head_dim;
  m->x = (uint16_t *)malloc(2 * c->hidden);
  m->norm = (uint16_t *)malloc(2 * c->hidden);
  m->q = (uint16_t *)malloc(2 * qd);
  m->k = (uint16_t *)malloc(2 * kvd);
  m->v = (uint16_t *)malloc(2 * kvd);
  m->attn = (uint16_t *)malloc(2 * qd);
  m->tmp = (uint16_t *)malloc(2 * c->hidden);
  m->gate = (uint16_t *)malloc(2 * (uint64_t)c->intermediate);
  m->up = (uint16_t *)malloc(2 * (uint64_t)c->intermediate);
  m->logits = (uint16_t *)malloc(2 * (uint64_t)c->vocab);
  return m;
}

void orc_qwen3_destroy(orc_qwen3 *m) {
  if (!m) return;
  for (uint32_t i = 0; i < m->c.layers * 11; ++i) free(m->w[i]);
  free(m->w);
  if (m->lm_head != m->embed) free(m->lm_head);
  free(m->embed); free(m->final_norm); free(m->kcache); free(m->vcache);
  free(m->cos_t); free(m->sin_t); free(m->x); free(m->norm); free(m->q);
  free(m->k); free(m->v); free(m->attn); free(m->tmp); free(m->gate);
  free(m->up); free(m->logits);
  free(m);
}

uint16_t *orc_qwen3_weight(orc_qwen3 *m, int kind, uint32_t layer) {
  if (kind == ORC_W_EMBED) return m->embed;
  if (kind == ORC_W_FINALNORM) return m->final_norm;
  if (kind == ORC_W_LMHEAD) return m->lm_head;
  return m->w[layer * 11 + kind];
}

const uint16_t *orc_qwen3_hidden(orc_qwen3 *m) { return m->x; }

static void gemv_bf16(const uint16_t *a, const uint16_t *x, uint16_t *y, uint32_t rows,
                      uint32_t cols) {
  orc_gemv_canonical(a, x, y, rows, cols, cols, 0);
}

/* qwen3/main.cpp:159-226 (Engine::decode), shape-parameterised; lm_head is
 * the embedding when the config is tied. */
uint32_t orc_qwen3_decode(orc_qwen3 *m, uint32_t token, uint32_t position,
                          uint16_t *logits) {
  const orc_qwen3_config *c = &m->c;
  const uint32_t H = c->hidden, D = c->head_dim, group = c->heads / c->kv_heads;
  memcpy(m->x, m->embed + (uint64_t)token * H, 2 * (uint64_t)H);
  const uint16_t *cos_row = m->cos_t + (uint64_t)position * D;
  const uint16_t *sin_row = m->sin_t + (uint64_t)position * D;
  for (uint32_t l = 0; l < c->layers; ++l) {
    uint16_t **w = m->w + (uint64_t)l * 11;
    orc_rmsnorm(m->x, w[ORC_W_INNORM], m->norm, H, c->rms_eps);
    gemv_bf16(w[ORC_W_Q], m->norm, m->q, c->heads * D, H);
    gemv_bf16(w[ORC_W_K], m->norm, m->k, c->kv_heads * D, H);
    gemv_bf16(w[ORC_W_V], m->norm, m->v, c->kv_heads * D, H);
    uint16_t *kc = m->kcache + (uint64_t)l * c->kv_heads * m->max_seq * D;
    uint16_t *vc = m->vcache + (uint64_t)l * c->kv_heads * m->max_seq * D;
    for (uint32_t g = 0; g < c->kv_heads; ++g) {
      orc_qk_norm_rope(m->k + g * D, w[ORC_W_KNORM], cos_row, sin_row, D, c->rms_eps);
      memcpy(kc + ((uint64_t)g * m->max_seq + position) * D, m->k + g * D, 2 * D);
      memcpy(vc + ((uint64_t)g * m->max_seq + position) * D, m->v + g * D, 2 * D);
    }
    for (uint32_t h = 0; h < c->heads; ++h) {
      const uint32_t g = h / group;
      orc_qk_norm_rope(m->q + h * D, w[ORC_W_QNORM], cos_row, sin_row, D, c->rms_eps);
      orc_attention_head(m->q + h * D, kc + (uint64_t)g * m->max_seq * D,
                         vc + (uint64_t)g * m->max_seq * D, D, position + 1, D,
                         m->attn + h * D);
    }
    gemv_bf16(w[ORC_W_O], m->attn, m->tmp, H, c->heads * D);
    orc_add(m->x, m->tmp, H);
    orc_rmsnorm(m->x, w[ORC_W_POSTNORM], m->norm, H, c->rms_eps);
    gemv_bf16(w[ORC_W_GATE], m->norm, m->gate, c->intermediate, H);
    gemv_bf16(w[ORC_W_UP], m->norm, m->up, c->intermediate, H);
    orc_silu_mul(m->gate, m->up, c->intermediate);
    gemv_bf16(w[ORC_W_DOWN], m->gate, m->tmp, H, c->intermediate);
    orc_add(m->x, m->tmp, H);
  }
  orc_rmsnorm(m->x, m->final_norm, m->norm, H, c->rms_eps);
  gemv_bf16(m->lm_head, m->norm, m->logits, c->vocab, H);
  if (logits) memcpy(logits, m->logits, 2 * (uint64_t)c->vocab);
  return orc_argmax(m->logits, c->vocab);
}

/* qwen3/main.cpp:342-352: the prompt goes through decode one position at a
 * time; generated token i is the argmax of the step before it; EOS
 * (151645, 151643; qwen3/model.hpp:19-20) stops the loop when requested. */
uint32_t orc_qwen3_generate(orc_qwen3 *m, const uint32_t *prompt, uint32_t n_prompt,
                            uint32_t max_new, uint32_t stop_on_eos, uint32_t *out,
                            uint16_t *logits_steps, uint32_t n_logit_steps) {
  uint32_t next = 0;
  const uint32_t V = m->c.vocab;
  for (uint32_t p = 0; p < n_prompt; ++p)
    next = orc_qwen3_decode(m, prompt[p], p,
                            (p + 1 == n_prompt && n_logit_steps) ? logits_steps : NULL);
  uint32_t produced = 0;
  for (uint32_t i = 0; i < max_new; ++i) {
    out[produced++] = next;
    if (next == 0xffffffffu) break;
    if (stop_on_eos && (next == 151645u || next == 151643u)) break;
    if (i + 1 != max_new)
      next = orc_qwen3_decode(m, next, n_prompt + i,
                              (i + 1 < n_logit_steps) ? logits_steps + (uint64_t)(i + 1) * V
                                                      : NULL);
  }
  return produced;
}
