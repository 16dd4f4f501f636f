/*
 * bf16 GEMV CPU oracle (the tied LM head) -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference's CPU check of the plain bf16 GEMV. Loaded only by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
 * checker; the product library never links or calls it.
 *
 * Pinning status:
 *   orc_bf16_fixture   known-answer LCG values vs an independent Python
 *                      restatement of tests/cuda/test_bf16_gemv.cpp:44-57
 *   orc_bf16_gemv      brute-force numpy fp32 sequential loop on tiny shapes
 *                      (bit-exact); fp64 bound at every shape; closed forms
 *                      (zero row -> +0, one-hot x -> bf16 of the weight,
 *                      sign flip)
 *   orc_bf16_gemv_f64  numpy float64 matmul of the bf16 values (exact
 *                      products, fp64 sum)
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <time.h>

#include "w4a16_oracle.h"

/* tests/cuda/test_bf16_gemv.cpp:44-57: s = s * 1664525 + 1013904223;
 * value = (s >> 8) * 2^-23 - 1 in [-1, 1), stored as bf16 RNE. W (N*K
 * values, row-major) is drawn first, then x (K values). */
void orc_bf16_fixture(uint32_t seed, int64_t N, int64_t K, uint16_t* W, uint16_t* X) {
  uint32_t s = seed;
  for (int64_t e = 0; e < N * K; ++e) {
    s = s * 1664525u + 1013904223u;
    const float v = (float)(s >> 8) * (2.0f / (float)(1u << 24)) - 1.0f;
    W[e] = orc_f32_to_bf16_rne(v);
  }
  for (int64_t k = 0; k < K; ++k) {
    s = s * 1664525u + 1013904223u;
    const float v = (float)(s >> 8) * (2.0f / (float)(1u << 24)) - 1.0f;
    X[k] = orc_f32_to_bf16_rne(v);
  }
}

/* ref_gemv_bf16 of tests/cuda/test_bf16_gemv.cpp:62-73 (and the batched
 * form, batch_decode.h:69-79): per output a sequential fp32 loop
 * acc += f32(W[n,k]) * f32(x[m,k]) over k ascending, one bf16 RNE. */
void orc_bf16_gemv_rows(const uint16_t* W, const uint16_t* X, uint16_t* Y, int64_t N, int64_t K,
                        int64_t M, int64_t n0, int64_t n1) {
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t* xr = X + m * K;
    for (int64_t n = n0; n < n1; ++n) {
      const uint16_t* wr = W + n * K;
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float p = orc_bf16_to_f32(wr[k]) * orc_bf16_to_f32(xr[k]);
        acc += p;
      }
      Y[m * N + n] = orc_f32_to_bf16_rne(acc);
    }
  }
}

void orc_bf16_gemv(const uint16_t* W, const uint16_t* X, uint16_t* Y, int64_t N, int64_t K,
                   int64_t M) {
  orc_bf16_gemv_rows(W, X, Y, N, K, M, 0, N);
}

typedef struct {
  const uint16_t* W;
  const uint16_t* X;
  uint16_t* Y;
  int64_t N, K, M, n0, n1;
} orc_bf16_job;

static void* orc_bf16_job_run(void* p) {
  orc_bf16_job* j = (orc_bf16_job*)p;
  orc_bf16_gemv_rows(j->W, j->X, j->Y, j->N, j->K, j->M, j->n0, j->n1);
  return NULL;
}

/* Output rows partitioned over threads; bit-identical to orc_bf16_gemv. */
void orc_bf16_gemv_mt(const uint16_t* W, const uint16_t* X, uint16_t* Y, int64_t N, int64_t K,
                      int64_t M, int nthreads) {
  if (nthreads <= 1 || N < 2) {
    orc_bf16_gemv(W, X, Y, N, K, M);
    return;
  }
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  orc_bf16_job jobs[256];
  const int64_t per = (N + nthreads - 1) / nthreads;
  int used = 0;
  for (int t = 0; t < nthreads; ++t) {
    const int64_t n0 = t * per;
    int64_t n1 = n0 + per;
    if (n0 >= N) break;
    if (n1 > N) n1 = N;
    jobs[t] = (orc_bf16_job){W, X, Y, N, K, M, n0, n1};
    pthread_create(&th[t], NULL, orc_bf16_job_run, &jobs[t]);
    ++used;
  }
  for (int t = 0; t < used; ++t) pthread_join(th[t], NULL);
}

/* fp64 sum of the exact products, and the sum of their magnitudes. */
void orc_bf16_gemv_f64(const uint16_t* W, const uint16_t* X, double* Y, double* Yabs, int64_t N,
                       int64_t K, int64_t M) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0, aacc = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double t = (double)orc_bf16_to_f32(W[n * K + k]) * (double)orc_bf16_to_f32(X[m * K + k]);
        acc += t;
        aacc += fabs(t);
      }
      Y[m * N + n] = acc;
      if (Yabs) Yabs[m * N + n] = aacc;
    }
  }
}

double orc_time_bf16_gemv(const uint16_t* W, const uint16_t* X, uint16_t* Y, int64_t N, int64_t K,
                          int64_t M, int nthreads, int iters) {
  struct timespec t0, t1;
  orc_bf16_gemv_mt(W, X, Y, N, K, M, nthreads);
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int i = 0; i < iters; ++i) orc_bf16_gemv_mt(W, X, Y, N, K, M, nthreads);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  const double dt = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
  return dt / (iters > 0 ? iters : 1);
}
