/*
 * W4A16 CPU oracle -- TEST INFRASTRUCTURE ONLY (see w4a16_oracle.h).
 *
 * Restates, in plain C, the reference's CPU-side W4A16 contract:
 *   - nibble unpack           include/cudalm/weight_loader.h:102-119
 *   - quantizer               tools/common/w4a16_quant.py:25-60,
 *                             docs/weight_format.md:135-153
 *   - dequant                 tools/common/w4a16_quant.py:74-82
 *   - ref_gemv_bf16           tests/cuda/test_int4_gemv_bf16.cpp:54-69
 *   - seeded fixtures         tests/cuda/test_int4_gemv_bf16.cpp:32-88,
 *                             tests/cuda/test_w4a16_qwen35_optimized.cpp:54-135
 *   - fp16 / bf16 decode      include/cudalm/stage_compare.h:28-77
 * The fp32 -> fp16 / bf16 round-to-nearest-even encoders are written from the
 * IEEE-754 definition (the reference uses the CUDA intrinsics
 * __float2half_rn / __float2bfloat16_rn, which implement the same rounding).
 *
 * Build with -ffp-contract=off: the reference's CPU loop performs separate
 * fp32 multiplies and adds, and contraction into fma would change the bits.
 */
#include "w4a16_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* numeric formats                                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Bit-exact binary16 -> binary32 (stage_compare.h:28-55 semantics). */
float orc_fp16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      /* subnormal: value m * 2^-24; normalise */
      int exp = 127 - 15 + 1;
      while ((m & 0x400u) == 0) {
        m <<= 1;
        --exp;
      }
      m &= 0x3FFu;
      bits = sign | ((uint32_t)exp << 23) | (m << 13);
    }
  } else if (e == 0x1Fu) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
  }
  return u2f(bits);
}

/* binary32 -> binary16, round to nearest, ties to even (IEEE-754 4.3.1). */
uint16_t orc_f32_to_fp16_rne(float f) {
  const uint32_t x = f2u(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const int exp = (int)((x >> 23) & 0xFFu);
  const uint32_t mant = x & 0x7FFFFFu;
  if (exp == 0xFF) {
    if (mant) return (uint16_t)(sign | 0x7E00u | (mant >> 13));
    return (uint16_t)(sign | 0x7C00u);
  }
  const int e = exp - 127 + 15; /* biased half exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    /* result is subnormal (or zero): h = round(m * 2^(e-14)) */
    const uint32_t m = (exp == 0) ? mant : (mant | 0x800000u);
    const int s = 14 - e; /* >= 14 */
    if (s >= 32) return sign;
    uint32_t hm = m >> s;
    const uint32_t rem = m & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = mant >> 13;
  const uint32_t rem = mant & 0x1FFFu;
  uint32_t r = ((uint32_t)e << 10) + hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) ++r; /* carry may reach inf */
  return (uint16_t)(sign | r);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* binary32 -> bfloat16, round to nearest, ties to even; NaN stays quiet NaN. */
uint16_t orc_f32_to_bf16_rne(float f) {
  const uint32_t x = f2u(f);
  if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu))
    return (uint16_t)((x >> 16) | 0x40u);
  const uint32_t r = x + 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

void orc_fp16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_fp16_to_f32(in[i]);
}
void orc_f32_to_fp16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_fp16_rne(in[i]);
}
void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16_rne(in[i]);
}

/* ------------------------------------------------------------------------ */
/* int4 contract                                                            */
/* ------------------------------------------------------------------------ */

/* weight_loader.h:106-117: low nibble = k=2b, high nibble = k=2b+1,
 * 4-bit two's complement, sign-extended. */
void orc_unpack_byte(uint8_t b, int* lo, int* hi) {
  *lo = (int)(int8_t)(uint8_t)((b & 0x0Fu) << 4) >> 4;
  *hi = (int)(int8_t)b >> 4;
}

/* weight_loader.h:104-106 */
uint8_t orc_pack_byte(int lo, int hi) {
  return (uint8_t)(((hi & 0xF) << 4) | (lo & 0xF));
}

void orc_unpack(const uint8_t* W, int64_t N, int64_t K, int8_t* q) {
  const int64_t total = N * (K / 2);
  for (int64_t i = 0; i < total; ++i) {
    int lo, hi;
    orc_unpack_byte(W[i], &lo, &hi);
    q[2 * i] = (int8_t)lo;
    q[2 * i + 1] = (int8_t)hi;
  }
}

/* w4a16_quant.py:74-82: w = q * f32(scale_fp16[n, k/128]), exact in fp32. */
void orc_dequant(const uint8_t* W, const uint16_t* S, int64_t N, int64_t K,
                 float* out) {
  const int64_t G = K / 128;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t b = 0; b < K / 2; ++b) {
      int lo, hi;
      orc_unpack_byte(W[n * (K / 2) + b], &lo, &hi);
      const float s = orc_fp16_to_f32(S[n * G + (b >> 6)]);
      out[n * K + 2 * b] = (float)lo * s;
      out[n * K + 2 * b + 1] = (float)hi * s;
    }
  }
}

/* w4a16_quant.py:25-60 (contract docs/weight_format.md:135-153):
 * per (n, g): amax over 128 fp32 values; scale32 = amax / 7 (fp32 divide);
 * q = clamp(rne(w / scale32), -7, 7); all-zero group -> scale 0, q 0;
 * stored scale = fp16_rne(scale32). Returns 0, or -1 on bad shape/non-finite. */
int orc_quantize(const float* Wf, int64_t N, int64_t K, uint8_t* Wp,
                 uint16_t* S) {
  if (N < 1 || K <= 0 || K % 128 != 0) return -1;
  const int64_t G = K / 128;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t g = 0; g < G; ++g) {
      const float* w = Wf + n * K + g * 128;
      float amax = 0.0f;
      for (int i = 0; i < 128; ++i) {
        if (!isfinite(w[i])) return -1;
        const float a = fabsf(w[i]);
        if (a > amax) amax = a;
      }
      const float scale32 = amax / 7.0f;
      const int zero = (scale32 == 0.0f);
      int q[128];
      for (int i = 0; i < 128; ++i) {
        if (zero) {
          q[i] = 0;
          continue;
        }
        float r = nearbyintf(w[i] / scale32); /* round-half-to-even */
        if (r > 7.0f) r = 7.0f;
        if (r < -7.0f) r = -7.0f;
        q[i] = (int)r;
      }
      for (int i = 0; i < 64; ++i)
        Wp[n * (K / 2) + g * 64 + i] = orc_pack_byte(q[2 * i], q[2 * i + 1]);
      S[n * G + g] = orc_f32_to_fp16_rne(scale32);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* GEMV                                                                     */
/* ------------------------------------------------------------------------ */

/* test_int4_gemv_bf16.cpp:54-69 (ref_gemv_bf16), applied to each activation
 * row m (batch_decode.cu:99-105: row m uses x + m*K and writes y + m*N).
 * Per output: fp32 acc, k ascending, lo before hi, each term (q * s) * x,
 * one bf16 RNE store. */
static void gemv_acc_rows(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                          uint16_t* Y, float* Yacc, int64_t N, int64_t K, int64_t M,
                          int64_t n_begin, int64_t n_end) {
  const int64_t G = K / 128;
  float* xf = (float*)malloc(sizeof(float) * (size_t)K);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t k = 0; k < K; ++k) xf[k] = orc_bf16_to_f32(X[m * K + k]);
    for (int64_t n = n_begin; n < n_end; ++n) {
      const uint8_t* wrow = W + n * (K / 2);
      const uint16_t* srow = S + n * G;
      float acc = 0.0f;
      for (int64_t b = 0; b < K / 2; ++b) {
        const float s = orc_fp16_to_f32(srow[b >> 6]);
        int lo, hi;
        orc_unpack_byte(wrow[b], &lo, &hi);
        acc += (float)lo * s * xf[2 * b];
        acc += (float)hi * s * xf[2 * b + 1];
      }
      if (Y) Y[m * N + n] = orc_f32_to_bf16_rne(acc);
      if (Yacc) Yacc[m * N + n] = acc;
    }
  }
  free(xf);
}

void orc_gemv_bf16_rows(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                        uint16_t* Y, int64_t N, int64_t K, int64_t M,
                        int64_t n_begin, int64_t n_end) {
  gemv_acc_rows(W, S, X, Y, NULL, N, K, M, n_begin, n_end);
}

void orc_gemv_bf16(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                   uint16_t* Y, int64_t N, int64_t K, int64_t M) {
  orc_gemv_bf16_rows(W, S, X, Y, N, K, M, 0, N);
}

typedef struct {
  const uint8_t* W;
  const uint16_t* S;
  const uint16_t* X;
  uint16_t* Y;
  int64_t N, K, M, n0, n1;
  float* Yacc;
} orc_job;

static void* orc_job_run(void* p) {
  orc_job* j = (orc_job*)p;
  gemv_acc_rows(j->W, j->S, j->X, j->Y, j->Yacc, j->N, j->K, j->M, j->n0, j->n1);
  return NULL;
}

/* Same arithmetic, output rows partitioned over threads (bit-identical to
 * the single-thread call: every output keeps its own sequential k loop). */
static void gemv_acc_mt(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y,
                        float* Yacc, int64_t N, int64_t K, int64_t M, int nthreads) {
  if (nthreads <= 1 || N < 2) {
    gemv_acc_rows(W, S, X, Y, Yacc, N, K, M, 0, N);
    return;
  }
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  orc_job jobs[256];
  const int64_t per = (N + nthreads - 1) / nthreads;
  int used = 0;
  for (int t = 0; t < nthreads; ++t) {
    const int64_t n0 = t * per;
    int64_t n1 = n0 + per;
    if (n0 >= N) break;
    if (n1 > N) n1 = N;
    jobs[t] = (orc_job){W, S, X, Y, N, K, M, n0, n1, Yacc};
    pthread_create(&th[t], NULL, orc_job_run, &jobs[t]);
    ++used;
  }
  for (int t = 0; t < used; ++t) pthread_join(th[t], NULL);
}

void orc_gemv_bf16_mt(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                      uint16_t* Y, int64_t N, int64_t K, int64_t M,
                      int nthreads) {
  gemv_acc_mt(W, S, X, Y, NULL, N, K, M, nthreads);
}

/* The same loop's fp32 accumulator before its bf16 rounding: the
 * "fp32-accumulated reference" a kernel output is measured against in bf16
 * ulps. orc_gemv_bf16 == bf16_rne(orc_gemv_f32acc) bit for bit. */
void orc_gemv_f32acc_mt(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                        float* Yacc, int64_t N, int64_t K, int64_t M, int nthreads) {
  gemv_acc_mt(W, S, X, NULL, Yacc, N, K, M, nthreads);
}

/* ref_gemv of tests/cuda/test_int4_gemv.cpp:49-63 (fp16 activations and
 * output): per output a sequential fp32 loop over bytes b, adding
 * (lo * s) * x[2b] then (hi * s) * x[2b+1], one fp16 RNE at the end. */
void orc_gemv_f16(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                  uint16_t* Y, int64_t N, int64_t K, int64_t M) {
  const int64_t G = K / 128;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      const uint8_t* wrow = W + n * (K / 2);
      const uint16_t* srow = S + n * G;
      float acc = 0.0f;
      for (int64_t b = 0; b < K / 2; ++b) {
        const float s = orc_fp16_to_f32(srow[b >> 6]);
        int lo, hi;
        orc_unpack_byte(wrow[b], &lo, &hi);
        acc += (float)lo * s * orc_fp16_to_f32(X[m * K + 2 * b]);
        acc += (float)hi * s * orc_fp16_to_f32(X[m * K + 2 * b + 1]);
      }
      Y[m * N + n] = orc_f32_to_fp16_rne(acc);
    }
  }
}

/* fp64 sum of the exact fp32 terms with fp16 activations, and |terms|. */
void orc_gemv_f16_f64(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                      double* Y, double* Yabs, int64_t N, int64_t K, int64_t M) {
  const int64_t G = K / 128;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0, aacc = 0.0;
      for (int64_t b = 0; b < K / 2; ++b) {
        const double s = (double)orc_fp16_to_f32(S[n * G + (b >> 6)]);
        int lo, hi;
        orc_unpack_byte(W[n * (K / 2) + b], &lo, &hi);
        const double t0 = (double)lo * s * (double)orc_fp16_to_f32(X[m * K + 2 * b]);
        const double t1 = (double)hi * s * (double)orc_fp16_to_f32(X[m * K + 2 * b + 1]);
        acc += t0 + t1;
        aacc += fabs(t0) + fabs(t1);
      }
      Y[m * N + n] = acc;
      if (Yabs) Yabs[m * N + n] = aacc;
    }
  }
}

/* fp64 accumulation of the exact fp32 terms (q*s)*x; also returns the sum
 * of |terms| (the scale of the accumulated rounding error). */
void orc_gemv_f64(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                  double* Y, double* Yabs, int64_t N, int64_t K, int64_t M) {
  const int64_t G = K / 128;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0, aacc = 0.0;
      for (int64_t b = 0; b < K / 2; ++b) {
        const double s = (double)orc_fp16_to_f32(S[n * G + (b >> 6)]);
        int lo, hi;
        orc_unpack_byte(W[n * (K / 2) + b], &lo, &hi);
        const double t0 = (double)lo * s * (double)orc_bf16_to_f32(X[m * K + 2 * b]);
        const double t1 =
            (double)hi * s * (double)orc_bf16_to_f32(X[m * K + 2 * b + 1]);
        acc += t0 + t1;
        aacc += fabs(t0) + fabs(t1);
      }
      Y[m * N + n] = acc;
      if (Yabs) Yabs[m * N + n] = aacc;
    }
  }
}

/* orc_gemv_f64 with the output rows n partitioned over threads (each
 * output keeps its own sequential k loop, so the values are identical to
 * the single-thread call). Test infrastructure for large traversals. */
typedef struct {
  const uint8_t* W;
  const uint16_t* S;
  const uint16_t* X;
  double *Y, *Yabs;
  int64_t N, K, M, n0, n1;
} orc_f64_job;

static void* orc_f64_run(void* p) {
  orc_f64_job* j = (orc_f64_job*)p;
  const int64_t G = j->K / 128, n = j->n1 - j->n0;
  double* y = (double*)malloc(sizeof(double) * (size_t)(j->M * n));
  double* a = (double*)malloc(sizeof(double) * (size_t)(j->M * n));
  orc_gemv_f64(j->W + j->n0 * (j->K / 2), j->S + j->n0 * G, j->X, y, a, n, j->K, j->M);
  for (int64_t m = 0; m < j->M; ++m)
    for (int64_t r = 0; r < n; ++r) {
      j->Y[m * j->N + j->n0 + r] = y[m * n + r];
      if (j->Yabs) j->Yabs[m * j->N + j->n0 + r] = a[m * n + r];
    }
  free(y);
  free(a);
  return NULL;
}

void orc_gemv_f64_mt(const uint8_t* W, const uint16_t* S, const uint16_t* X, double* Y,
                     double* Yabs, int64_t N, int64_t K, int64_t M, int nthreads) {
  if (nthreads <= 1 || N < 2) {
    orc_gemv_f64(W, S, X, Y, Yabs, N, K, M);
    return;
  }
  if (nthreads > 64) nthreads = 64;
  pthread_t th[64];
  orc_f64_job jobs[64];
  const int64_t per = (N + nthreads - 1) / nthreads;
  int used = 0;
  for (int t = 0; t < nthreads; ++t) {
    const int64_t n0 = t * per, n1 = n0 + per < N ? n0 + per : N;
    if (n0 >= n1) break;
    jobs[t] = (orc_f64_job){W, S, X, Y, Yabs, N, K, M, n0, n1};
    pthread_create(&th[t], NULL, orc_f64_run, &jobs[t]);
    ++used;
  }
  for (int t = 0; t < used; ++t) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* seeded fixtures                                                          */
/* ------------------------------------------------------------------------ */

/* test_int4_gemv_bf16.cpp:32-42 (struct Rng): xorshift32 13/17/5,
 * seed 0 replaced by 0x9e3779b9. */
uint32_t orc_xorshift32_next(uint32_t* s) {
  uint32_t x = *s;
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  *s = x;
  return x;
}

void orc_xorshift32_fill(uint32_t seed, uint32_t* out, size_t n) {
  uint32_t s = seed ? seed : 0x9e3779b9u;
  for (size_t i = 0; i < n; ++i) out[i] = orc_xorshift32_next(&s);
}

static inline float rng_n01(uint32_t* s) {
  return (float)orc_xorshift32_next(s) * (2.0f / 4294967296.0f) - 1.0f;
}
static inline uint16_t rng_scale(uint32_t* s) {
  const float u = (float)orc_xorshift32_next(s);
  return orc_f32_to_fp16_rne(0.001f + 0.02f * u * (1.0f / 4294967296.0f));
}

/* test_int4_gemv_bf16.cpp:77-88 (make_fixture): W random bytes, S in
 * [0.001, 0.021) as fp16, x in [-1, 1) as bf16; drawn in that order. */
void orc_fixture_gemv(uint32_t seed, int64_t N, int64_t K, uint8_t* W,
                      uint16_t* S, uint16_t* X) {
  uint32_t s = seed ? seed : 0x9e3779b9u;
  for (int64_t i = 0; i < N * (K / 2); ++i) W[i] = (uint8_t)orc_xorshift32_next(&s);
  for (int64_t i = 0; i < N * (K / 128); ++i) S[i] = rng_scale(&s);
  for (int64_t i = 0; i < K; ++i) X[i] = orc_f32_to_bf16_rne(rng_n01(&s));
}

/* tests/cuda/test_int4_gemv.cpp:70-83 (the fp16 twin's fixture): the same
 * draws as orc_fixture_gemv with x stored as fp16 RNE. */
void orc_fixture_gemv_f16(uint32_t seed, int64_t N, int64_t K, uint8_t* W,
                          uint16_t* S, uint16_t* X) {
  uint32_t s = seed ? seed : 0x9e3779b9u;
  for (int64_t i = 0; i < N * (K / 2); ++i) W[i] = (uint8_t)orc_xorshift32_next(&s);
  for (int64_t i = 0; i < N * (K / 128); ++i) S[i] = rng_scale(&s);
  for (int64_t i = 0; i < K; ++i) X[i] = orc_f32_to_fp16_rne(rng_n01(&s));
}

/* test_w4a16_qwen35_optimized.cpp:66-135 (make_fixture with InputKind).
 * Where the reference draws two numbers inside one unsequenced C++
 * expression (the kSmall / kBoundary weight bytes), the left operand is
 * drawn first. X holds B rows of K. */
void orc_fixture_kind(int kind, uint32_t seed, int64_t N, int64_t K,
                      int64_t B, uint8_t* W, uint16_t* S, uint16_t* X) {
  static const uint8_t kNib[8] = {0x7, 0x9, 0x8, 0x0, 0xF, 0x7, 0x8, 0xF};
  uint32_t s = seed ? seed : 0x9e3779b9u;
  for (int64_t i = 0; i < N * (K / 2); ++i) {
    uint8_t b;
    if (kind == ORC_KIND_ZERO) {
      b = 0;
    } else if (kind == ORC_KIND_SMALL) {
      const uint32_t a = orc_xorshift32_next(&s) % 3u;
      const uint32_t c = orc_xorshift32_next(&s) % 3u;
      b = (uint8_t)(a | (c << 4));
    } else if (kind == ORC_KIND_BOUNDARY) {
      const uint8_t a = kNib[orc_xorshift32_next(&s) % 8u];
      const uint8_t c = kNib[orc_xorshift32_next(&s) % 8u];
      b = (uint8_t)(a | (c << 4));
    } else {
      b = (uint8_t)orc_xorshift32_next(&s);
    }
    W[i] = b;
  }
  for (int64_t i = 0; i < N * (K / 128); ++i) {
    if (kind == ORC_KIND_BOUNDARY && orc_xorshift32_next(&s) % 5u == 0) {
      S[i] = orc_f32_to_fp16_rne(0.0f);
      continue;
    }
    S[i] = rng_scale(&s);
  }
  for (int64_t i = 0; i < B * K; ++i) {
    float v;
    if (kind == ORC_KIND_ZERO) {
      v = 0.0f;
    } else if (kind == ORC_KIND_SMALL) {
      v = 0.01f * (float)orc_xorshift32_next(&s) * (1.0f / 4294967296.0f) - 0.005f;
    } else if (kind == ORC_KIND_MIXED_SIGN) {
      if (orc_xorshift32_next(&s) & 1u)
        v = -rng_n01(&s);
      else
        v = rng_n01(&s);
    } else {
      v = rng_n01(&s);
    }
    X[i] = orc_f32_to_bf16_rne(v);
  }
}

/* Synthetic N(0, sigma) source for the benchmark configs: splitmix64 stream
 * (Steele, Lea & Flood 2014) feeding the Box-Muller transform in double,
 * rounded once to fp32. Element i depends only on (seed, i). */
static inline uint64_t splitmix64(uint64_t* x) {
  uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static void normal_block(uint64_t seed, float sigma, float* out, size_t begin,
                         size_t end) {
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = begin & ~(size_t)1;
  uint64_t st = seed + (uint64_t)(i / 2) * 2u * 0x9E3779B97F4A7C15ull;
  for (; i < end; i += 2) {
    const uint64_t a = splitmix64(&st), b = splitmix64(&st);
    const double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = ((double)(b >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    if (i >= begin) out[i] = (float)(sigma * r * cos(two_pi * u2));
    if (i + 1 < end) out[i + 1] = (float)(sigma * r * sin(two_pi * u2));
  }
}

typedef struct {
  uint64_t seed;
  float sigma;
  float* out;
  size_t b, e;
} normal_job;

static void* normal_run(void* p) {
  normal_job* j = (normal_job*)p;
  normal_block(j->seed, j->sigma, j->out, j->b, j->e);
  return NULL;
}

void orc_synth_normal_f32(uint64_t seed, float sigma, float* out, size_t n) {
  int nt = orc_hardware_threads();
  if (nt > 64) nt = 64;
  if (n < (1u << 20)) nt = 1;
  pthread_t th[64];
  normal_job jobs[64];
  size_t per = ((n + nt - 1) / nt + 1) & ~(size_t)1; /* even split points */
  int used = 0;
  for (int t = 0; t < nt; ++t) {
    size_t b = (size_t)t * per, e = b + per;
    if (b >= n) break;
    if (e > n) e = n;
    jobs[t] = (normal_job){seed, sigma, out, b, e};
    pthread_create(&th[t], NULL, normal_run, &jobs[t]);
    ++used;
  }
  for (int t = 0; t < used; ++t) pthread_join(th[t], NULL);
}

typedef struct {
  const float* w;
  uint8_t* Wp;
  uint16_t* S;
  int64_t n0, n1, K;
  int rc;
} quant_job;

static void* quant_run(void* p) {
  quant_job* j = (quant_job*)p;
  const int64_t G = j->K / 128;
  j->rc = orc_quantize(j->w + j->n0 * j->K, j->n1 - j->n0, j->K,
                       j->Wp + j->n0 * (j->K / 2), j->S + j->n0 * G);
  return NULL;
}

/* BASELINE weights: W ~ N(0, sigma) in fp32, then the reference quantizer. */
int orc_synth_w4a16(uint64_t seed, float sigma, int64_t N, int64_t K,
                    uint8_t* W, uint16_t* S) {
  if (N < 1 || K <= 0 || K % 128 != 0) return -1;
  float* wf = (float*)malloc(sizeof(float) * (size_t)(N * K));
  if (!wf) return -2;
  orc_synth_normal_f32(seed, sigma, wf, (size_t)(N * K));
  int nt = orc_hardware_threads();
  if (nt > 64) nt = 64;
  if (N < 256) nt = 1;
  pthread_t th[64];
  quant_job jobs[64];
  const int64_t per = (N + nt - 1) / nt;
  int used = 0;
  for (int t = 0; t < nt; ++t) {
    int64_t n0 = t * per, n1 = n0 + per;
    if (n0 >= N) break;
    if (n1 > N) n1 = N;
    jobs[t] = (quant_job){wf, W, S, n0, n1, K, 0};
    pthread_create(&th[t], NULL, quant_run, &jobs[t]);
    ++used;
  }
  int rc = 0;
  for (int t = 0; t < used; ++t) {
    pthread_join(th[t], NULL);
    if (jobs[t].rc) rc = jobs[t].rc;
  }
  free(wf);
  return rc;
}

/* BASELINE activations: X ~ N(0, 1), rounded to bf16 (RNE). */
void orc_synth_act_bf16(uint64_t seed, int64_t M, int64_t K, uint16_t* X) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  orc_synth_normal_f32(seed, 1.0f, xf, (size_t)(M * K));
  orc_f32_to_bf16_array(xf, X, (size_t)(M * K));
  free(xf);
}

/* ------------------------------------------------------------------------ */
/* CPU baseline timing                                                      */
/* ------------------------------------------------------------------------ */

int orc_hardware_threads(void) {
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

/* Seconds per call, averaged over `iters` calls after one warm-up call. */
double orc_time_gemv_bf16(const uint8_t* W, const uint16_t* S,
                          const uint16_t* X, uint16_t* Y, int64_t N, int64_t K,
                          int64_t M, int nthreads, int iters) {
  struct timespec t0, t1;
  orc_gemv_bf16_mt(W, S, X, Y, N, K, M, nthreads);
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int i = 0; i < iters; ++i) orc_gemv_bf16_mt(W, S, X, Y, N, K, M, nthreads);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  const double dt = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
  return dt / (iters > 0 ? iters : 1);
}
