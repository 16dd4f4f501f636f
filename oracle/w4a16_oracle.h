/*
 * W4A16 CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference's CPU W4A16 path, used as the checker
 * for the HIP kernels. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product library never links
 * or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the reference tree).
 *
 * Pinning status (what independent check fixes each function):
 *   orc_unpack_byte      exhaustive 256-byte table vs the closed form and the
 *                        pack/unpack round trip over [-8,7]^2
 *                        (tests/cpu/test_weight_file.cpp:212-225)
 *   orc_fp16_to_f32      all 65536 patterns vs numpy float16 (IEEE binary16)
 *   orc_f32_to_fp16_rne  2^20 sampled + edge patterns vs numpy astype(float16)
 *   orc_f32_to_bf16_rne  sampled + edge patterns vs torch bfloat16 conversion
 *   orc_dequant          q * f32(s) over all 16 q x all finite fp16 scales vs
 *                        numpy float32 products
 *   orc_quantize         invariants of tests/cpu/test_weights_crosslang.cpp:
 *                        58-100 + an independent torch restatement
 *   orc_gemv_bf16        brute-force fp32 sequential loop in numpy for tiny
 *                        shapes (bit-exact), fp64 matmul bound at all shapes,
 *                        closed forms (zero row, one-hot x, linearity, sign)
 *   orc_gemv_f32acc_mt   brute-force fp32 accumulator in numpy (bit-exact) and
 *                        bf16_rne of it == orc_gemv_bf16 at every test shape
 *   orc_gemv_f64         numpy float64 matmul of the dequantized weights
 *   orc_gemv_f16         as orc_gemv_bf16, with numpy float16 activations and
 *                        output (brute force bit-exact, fp64 bound, closed
 *                        forms); orc_gemv_f16_f64 as orc_gemv_f64
 *   orc_rng_*            xorshift32 known-answer sequence vs a Python restatement
 */
#ifndef CUDALM_W4A16_ORACLE_H
#define CUDALM_W4A16_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numeric formats ---------------------------------------------------- */
float orc_fp16_to_f32(uint16_t h);
uint16_t orc_f32_to_fp16_rne(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16_rne(float f);
void orc_fp16_to_f32_array(const uint16_t* in, float* out, size_t n);
void orc_f32_to_fp16_array(const float* in, uint16_t* out, size_t n);
void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n);

/* ---- int4 contract ------------------------------------------------------ */
void orc_unpack_byte(uint8_t b, int* lo, int* hi);
uint8_t orc_pack_byte(int lo, int hi);
void orc_unpack(const uint8_t* W, int64_t N, int64_t K, int8_t* q);
void orc_dequant(const uint8_t* W, const uint16_t* S, int64_t N, int64_t K,
                 float* out);
int orc_quantize(const float* Wf, int64_t N, int64_t K, uint8_t* Wp,
                 uint16_t* S);

/* ---- GEMV / GEMM -------------------------------------------------------- */
void orc_gemv_bf16(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                   uint16_t* Y, int64_t N, int64_t K, int64_t M);
void orc_gemv_bf16_rows(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                        uint16_t* Y, int64_t N, int64_t K, int64_t M,
                        int64_t n_begin, int64_t n_end);
void orc_gemv_bf16_mt(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                      uint16_t* Y, int64_t N, int64_t K, int64_t M,
                      int nthreads);
void orc_gemv_f32acc_mt(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                        float* Yacc, int64_t N, int64_t K, int64_t M, int nthreads);
void orc_gemv_f64_mt(const uint8_t* W, const uint16_t* S, const uint16_t* X, double* Y,
                     double* Yabs, int64_t N, int64_t K, int64_t M, int nthreads);
void orc_gemv_f64(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                  double* Y, double* Yabs, int64_t N, int64_t K, int64_t M);

void orc_gemv_f16(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                  uint16_t* Y, int64_t N, int64_t K, int64_t M);
void orc_gemv_f16_f64(const uint8_t* W, const uint16_t* S, const uint16_t* X,
                      double* Y, double* Yabs, int64_t N, int64_t K, int64_t M);

/* ---- seeded fixtures ---------------------------------------------------- */
uint32_t orc_xorshift32_next(uint32_t* state);
void orc_xorshift32_fill(uint32_t seed, uint32_t* out, size_t n);
enum {
  ORC_KIND_RANDOM = 0,
  ORC_KIND_ZERO = 1,
  ORC_KIND_SMALL = 2,
  ORC_KIND_MIXED_SIGN = 3,
  ORC_KIND_BOUNDARY = 4
};
void orc_fixture_gemv(uint32_t seed, int64_t N, int64_t K, uint8_t* W,
                      uint16_t* S, uint16_t* X);
void orc_fixture_gemv_f16(uint32_t seed, int64_t N, int64_t K, uint8_t* W,
                          uint16_t* S, uint16_t* X);
void orc_fixture_kind(int kind, uint32_t seed, int64_t N, int64_t K,
                      int64_t B, uint8_t* W, uint16_t* S, uint16_t* X);
void orc_synth_normal_f32(uint64_t seed, float sigma, float* out, size_t n);
int orc_synth_w4a16(uint64_t seed, float sigma, int64_t N, int64_t K,
                    uint8_t* W, uint16_t* S);
void orc_synth_act_bf16(uint64_t seed, int64_t M, int64_t K, uint16_t* X);

/* ---- bf16 GEMV (tied LM head), bf16_oracle.c --------------------------- */
void orc_bf16_fixture(uint32_t seed, int64_t N, int64_t K, uint16_t* W, uint16_t* X);
void orc_bf16_gemv(const uint16_t* W, const uint16_t* X, uint16_t* Y, int64_t N,
                   int64_t K, int64_t M);
void orc_bf16_gemv_rows(const uint16_t* W, const uint16_t* X, uint16_t* Y,
                        int64_t N, int64_t K, int64_t M, int64_t n0, int64_t n1);
void orc_bf16_gemv_mt(const uint16_t* W, const uint16_t* X, uint16_t* Y,
                      int64_t N, int64_t K, int64_t M, int nthreads);
void orc_bf16_gemv_f64(const uint16_t* W, const uint16_t* X, double* Y,
                       double* Yabs, int64_t N, int64_t K, int64_t M);
double orc_time_bf16_gemv(const uint16_t* W, const uint16_t* X, uint16_t* Y,
                          int64_t N, int64_t K, int64_t M, int nthreads,
                          int iters);

/* ---- SwiGLU element-wise stage, swiglu_oracle.c ------------------------ */
uint16_t orc_silu_bf16(uint16_t g_bits);
void orc_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* y, size_t n);

/* ---- timing helper for the CPU baseline --------------------------------- */
double orc_time_gemv_bf16(const uint8_t* W, const uint16_t* S,
                          const uint16_t* X, uint16_t* Y, int64_t N, int64_t K,
                          int64_t M, int nthreads, int iters);
int orc_hardware_threads(void);

#ifdef __cplusplus
}
#endif

#endif
