/*
 * cudalm_w4a16 -- C ABI of the MI355X (gfx950) W4A16 projection engine.
 *
 * Arithmetic contract (the reference's, include/cudalm/kernels/
 * int4_gemv_bf16.h:6-9,29-37):
 *
 *   y[m, n] = bf16_rne( sum_k q[n, k] * f32(scale_fp16[n, k / 128]) * f32(x[m, k]) )
 *
 *   weight : packed int4 [N, K/2] uint8, row-major. Low nibble of byte b is
 *            element k = 2b, high nibble is k = 2b+1, 4-bit two's complement.
 *   scale  : fp16 bit patterns [N, K/128], row-major (the stored fp16 scale
 *            is the contract, docs/weight_format.md:135-153).
 *   x      : bf16 bit patterns [M, K], row-major (M activation rows).
 *   y      : bf16 bit patterns [M, N], row-major.
 *
 * Accumulation is fp32; the output is rounded once to bf16 (round to
 * nearest even). Results are within 2 bf16 ulp of an fp32-accumulated
 * reference plus a floor for outputs that cancel (the tests state it).
 * Every entry point computes row m of a batched call bit-identically to a
 * single-row call on row m, whichever kernel (M = 1 stream, small-M tile,
 * prefill tile) and weight layout (file or prepacked) serves it.
 *
 * Ownership and threading: the caller owns every buffer. Entry points keep
 * no state, never synchronize, and enqueue asynchronously on `stream`.
 * Device pointers must be device-accessible; misaligned weight / x bases
 * are accepted (a byte-wise fallback kernel serves them), as the reference
 * requires (int4_gemv_bf16.h:39-45).
 *
 * Error model: each call returns 0 or a negative CUDALM_W4A16_E* code and
 * leaves the stream untouched on a precondition failure. The C++ wrappers
 * under include/cudalm/ turn a nonzero code into the reference's fatal
 * abort (cuda_check.h:53-63).
 */
#ifndef CUDALM_W4A16_H
#define CUDALM_W4A16_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CUDALM_W4A16_OK 0
#define CUDALM_W4A16_EINVAL (-1)  /* N < 1, M < 1, K <= 0 or K % 128 != 0 */
#define CUDALM_W4A16_ENULL (-2)   /* a required pointer is NULL */
#define CUDALM_W4A16_EALIGN (-3)  /* a prepacked buffer is not 16 B aligned */
#define CUDALM_W4A16_ELAUNCH (-4) /* the HIP runtime rejected a launch */
#define CUDALM_W4A16_ERANGE (-5)  /* sizes overflow the kernels' index range */
#define CUDALM_W4A16_EVARIANT (-6) /* unknown kernel variant id */

#define CUDALM_W4A16_GROUP 128

/* Library version (major * 10000 + minor * 100 + patch). */
int cudalm_w4a16_version(void);

/* Human-readable text for a return code. Never NULL. */
const char* cudalm_w4a16_strerror(int code);

/* y[M, N] = W4A16(weight, scale) applied to x[M, K], file weight layout.
 * Replaces int4_gemv_bf16 (M == 1; include/cudalm/kernels/
 * int4_gemv_bf16.h:46-48) and kernels::batch_int4_gemv_bf16 (M == B;
 * include/cudalm/kernels/batch_decode.h:61-63), and serves prefill chunks
 * (M >= 64), which the reference runs one token at a time. */
int cudalm_w4a16_gemv_bf16(const uint8_t* weight, const uint16_t* scale,
                           const uint16_t* x, uint16_t* y, int N, int K, int M,
                           hipStream_t stream);

/* Bytes of the prepacked (load-time repacked) form of an [N, K] weight,
 * G = K/128: ceil(N/16) * (G * 1024 + 256 * ceil(G/8)). Per 16-row tile:
 * G slabs of 1024 weight bytes (16 bytes per MFMA lane; each little-endian
 * dword of 8 nibbles stored rotated left by 3 bits), then the tile's
 * 16 rows of fp16 scales, each row padded to 16 * ceil(G/8) bytes.
 * 0 on invalid shape. */
size_t cudalm_w4a16_packed_bytes(int N, int K);

/* Load-time repack, device to device (stream-ordered). `packed` must hold
 * cudalm_w4a16_packed_bytes(N, K) bytes, 16 B aligned. The hook the
 * reference's loader would call next to its upload lambda
 * (src/runtime/weight_loader_v2.cpp:435-441). */
int cudalm_w4a16_repack(const uint8_t* weight, const uint16_t* scale,
                        void* packed, int N, int K, hipStream_t stream);

/* The same repack on host memory (for loaders that hold the file bytes on
 * the host before the upload). Byte-identical to cudalm_w4a16_repack. */
int cudalm_w4a16_repack_host(const uint8_t* weight, const uint16_t* scale,
                             void* packed, int N, int K);

/* y[M, N] from a prepacked weight. Bit-identical to cudalm_w4a16_gemv_bf16
 * on the file layout it was packed from. `packed` and `x` must be 16 B
 * aligned (x may not be: then EALIGN). */
int cudalm_w4a16_gemv_bf16_prepacked(const void* packed, const uint16_t* x,
                                     uint16_t* y, int N, int K, int M,
                                     hipStream_t stream);

/* Several projections that read the same activations x[M, K] (the
 * q/k/v, in_proj_qkv/z/b/a and gate/up groups of a decoder layer,
 * src/runtime/qwen35_deltanet.cpp:166-181,236-243 and
 * src/runtime/qwen35_full_attention.cpp:211-240), computed by one launch
 * when M <= 32 and x fits on chip, else one launch per projection. Each
 * y_j is bit-identical to the single-projection call. No counterpart in the
 * reference (it issues one launch per projection). */
#define CUDALM_W4A16_MAX_PROJ 8
typedef struct cudalm_w4a16_proj {
  const void* weight;    /* file layout [N, K/2] or prepacked */
  const uint16_t* scale; /* fp16 [N, K/128]; ignored when prepacked */
  uint16_t* y;           /* bf16 [M, N] */
  int N;
} cudalm_w4a16_proj;
int cudalm_w4a16_gemv_bf16_multi(const cudalm_w4a16_proj* projs, int count,
                                 const uint16_t* x, int K, int M, int prepacked,
                                 hipStream_t stream);

/* Stage chains: an ordered list of projection stages run by ONE persistent
 * launch, for the dependent projection sequence of a decode step
 * (src/runtime/qwen35_model.cpp:469-491 issues each projection as its own
 * launch; src/runtime/qwen35_deltanet.cpp:166-251). No counterpart in the
 * reference. A stage is up to 4 projections sharing x[M, K] (as in
 * cudalm_w4a16_gemv_bf16_multi); `dep` names an earlier stage (or -1) that
 * must have completed before this stage reads x, because x is that stage's
 * output or simply must follow it. A stage that writes a buffer another
 * stage reads must depend (directly or through deps) on every such reader.
 * Each output has the bits cudalm_w4a16_gemv_bf16 gives on the same inputs.
 * Limits: 1 <= M <= 32, K % 128 == 0 and K <= 4096, 1..4 projections per
 * stage, up to CUDALM_W4A16_MAX_STAGES stages; x and (prepacked) weights
 * 16 B aligned, y and scales 2 B aligned.
 *
 * The workspace is caller-owned device memory of
 * cudalm_w4a16_chain_workspace_bytes(n) bytes, 256 B aligned, holding the
 * plan, the completion flags and counters; one workspace serves one chain,
 * and launches sharing a workspace must not overlap in time.
 * cudalm_w4a16_chain_plan validates the stages, writes the plan into the
 * workspace and synchronizes `stream` (set-up time; not capturable);
 * cudalm_w4a16_chain_run is one kernel launch with no other stream work,
 * so it may be captured into a HIP graph and replayed. Every wait inside the
 * launch is bounded: on a timeout the chain finishes with unspecified
 * outputs and cudalm_w4a16_chain_status reports CUDALM_W4A16_ETIMEOUT. */
#define CUDALM_W4A16_MAX_STAGES 256
#define CUDALM_W4A16_ETIMEOUT (-10) /* a chain stage's wait passed its bound */
typedef struct cudalm_w4a16_stage {
  const cudalm_w4a16_proj* projs; /* 1..4 projections reading x */
  int count;
  const uint16_t* x; /* bf16 [M, K] */
  int K;
  int dep; /* earlier stage that must complete before x is read, or -1 */
  /* SwiGLU epilogue (NULL = none). When set, the stage has count == 2
   * projections of equal N, gate then up, and K <= 2048; it writes only
   *   act[m, n] = bf16( f32(bf16(silu(g))) * f32(u) )   (bf16 [M, N]),
   * g and u being the bits cudalm_w4a16_gemv_bf16 gives for gate and up,
   * i.e. what cudalm_w4a16_swiglu_bf16 writes; the projections' y are
   * ignored (may be NULL). A later stage with dep on this one may read act
   * as its x: the reference's gate -> up -> qwen35_silu_mul_bf16 -> down
   * sequence (src/runtime/qwen35_deltanet.cpp:236-251) as two stages of one
   * launch. No counterpart in the reference. */
  uint16_t* act;
} cudalm_w4a16_stage;
typedef struct cudalm_w4a16_chain { /* filled by cudalm_w4a16_chain_plan */
  void* workspace;
  int n_stages, M, prepacked, grid, gt_max;
} cudalm_w4a16_chain;
size_t cudalm_w4a16_chain_workspace_bytes(int n_stages);
int cudalm_w4a16_chain_plan(const cudalm_w4a16_stage* stages, int n_stages, int M, int prepacked,
                            void* workspace, size_t workspace_bytes, cudalm_w4a16_chain* chain,
                            hipStream_t stream);
int cudalm_w4a16_chain_run(const cudalm_w4a16_chain* chain, hipStream_t stream);
/* Synchronizes `stream`, then returns CUDALM_W4A16_ETIMEOUT (and clears
 * the record) if a wait of a run since the last call timed out, else 0. */
int cudalm_w4a16_chain_status(const cudalm_w4a16_chain* chain, hipStream_t stream);
/* Sets the bound of every wait of later runs of `chain`, in ticks of the
 * 100 MHz s_memrealtime counter (0 = the default, about 0.5 s), and
 * synchronizes `stream`; a new plan resets it to the default. A wait past
 * its bound gives up (its stage proceeds and every wave exits) and
 * cudalm_w4a16_chain_status then reports CUDALM_W4A16_ETIMEOUT. For callers
 * that prefer an early error to a long stall, and for tests of the timeout
 * path. No counterpart in the reference. */
int cudalm_w4a16_chain_set_wait_bound(const cudalm_w4a16_chain* chain, uint32_t ticks,
                                      hipStream_t stream);
/* plan + run in one call (not capturable: the plan synchronizes). */
int cudalm_w4a16_gemv_bf16_chain(const cudalm_w4a16_stage* stages, int n_stages, int M,
                                 int prepacked, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/* cudalm_w4a16_gemv_bf16_chain without a caller workspace, for callers that
 * cannot allocate device memory (code under graph-capture set-up, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The plan, flags and counters live in a file-scope device array
 * of the library (4,236,288 bytes per GPU, held until the process ends) that
 * holds up to CUDALM_W4A16_NOALLOC_MAX_STAGES stages; more stages return
 * CUDALM_W4A16_ERANGE. The call allocates nothing (no hipMalloc, no device
 * allocation of any library); it plans (copying the plan into that array and
 * synchronizing `stream`) and launches. Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU race, so serialize
 * them. Same limits and outputs as cudalm_w4a16_gemv_bf16_chain. */
#define CUDALM_W4A16_NOALLOC_MAX_STAGES 128
int cudalm_w4a16_gemv_bf16_chain_noalloc(const cudalm_w4a16_stage* stages, int n_stages, int M,
                                         int prepacked, hipStream_t stream);

/* fp16-activation twin of cudalm_w4a16_gemv_bf16: x and y are fp16 bit
 * patterns, y[m, n] = fp16_rne( sum_k q * f32(scale) * f32(x[m, k]) ) with
 * fp32 accumulation. Replaces int4_gemv (M == 1; include/cudalm/kernels/
 * int4_gemv.h:22-40); any M (chunks of up to 32 rows), row m bit-identical
 * to the M == 1 call. Misaligned weight / x bases take a byte-wise kernel. */
int cudalm_w4a16_gemv_f16(const uint8_t* weight, const uint16_t* scale,
                          const uint16_t* x, uint16_t* y, int N, int K, int M,
                          hipStream_t stream);

/* Same from the prepacked layout (packed and x 16 B aligned, else EALIGN);
 * bit-identical to cudalm_w4a16_gemv_f16 on the file layout. */
int cudalm_w4a16_gemv_f16_prepacked(const void* packed, const uint16_t* x,
                                    uint16_t* y, int N, int K, int M,
                                    hipStream_t stream);

/* SwiGLU MLP front half in one launch: the gate and up projections of the
 * same x[M, K] (both [N, K], file layout with scales or both prepacked)
 * and the epilogue
 *   y[m, n] = bf16( f32(bf16(silu(g))) * f32(u) ),  silu(g) = g / (1 + exp(-g))
 * on g = gate(x)[m, n] and u = up(x)[m, n] as bf16. g and u carry exactly
 * the bits of cudalm_w4a16_gemv_bf16 on each projection, and the epilogue
 * is cudalm_silu_mul_bf16's, so y equals the reference's three-step
 * sequence gate -> up -> qwen35_silu_mul_bf16
 * (src/runtime/qwen35_deltanet.cpp:236-247) run on this library, with no
 * intermediate buffers. Any M (processed in chunks of up to 32 rows); all
 * bases 16 B aligned (y: 2 B), else EALIGN. No counterpart in the
 * reference. */
int cudalm_w4a16_swiglu_bf16(const void* gate_weight, const uint16_t* gate_scale,
                             const void* up_weight, const uint16_t* up_scale,
                             const uint16_t* x, uint16_t* y, int N, int K, int M,
                             int prepacked, hipStream_t stream);

/* y[i] = bf16( f32(bf16(silu(f32(gate[i])))) * f32(up[i]) ) for i < n, bf16
 * bit patterns. Replaces kernels::qwen35_silu_mul_bf16
 * (include/cudalm/kernels/qwen35_kernels.h:146-154); any n and 2-byte
 * aligned bases (the reference requires n % 8 == 0 and 16 B bases). SiLU is
 * evaluated in fp32 with a correctly rounded divide and the device expf. */
int cudalm_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* y,
                         size_t n, hipStream_t stream);

/* Dequantize through the kernels' own nibble decoder: q_out[N, K] int8 and
 * w_out[N, K] = q * f32(scale) (either output may be NULL). The weight base
 * must be 4 B aligned. Equivalent to the reference's dequant_reference
 * (tools/common/w4a16_quant.py:74-82). */
int cudalm_w4a16_dequant_f32(const uint8_t* weight, const uint16_t* scale,
                             int8_t* q_out, float* w_out, int N, int K,
                             hipStream_t stream);

/* Kernel variants, for parity tests and benchmarks (the counterpart of the
 * reference's explicit per-variant launchers, include/cudalm/kernels/
 * int4_gemv_qwen35.h:59-83). Every variant is bit-identical per output to
 * the default dispatch except CUDALM_W4A16_VARIANT_BYTEWISE, which sums in
 * the reference's order and is within tolerance. */
#define CUDALM_W4A16_VARIANT_AUTO 0
#define CUDALM_W4A16_VARIANT_STREAM 1   /* M <= 32, x resident in LDS */
#define CUDALM_W4A16_VARIANT_TILE16 2   /* 16 columns per wave, K chunked */
#define CUDALM_W4A16_VARIANT_TILE32 3   /* 32 columns per wave, K chunked */
#define CUDALM_W4A16_VARIANT_PREFILL 4  /* prefill GEMM chosen by shape (M >= 33) */
#define CUDALM_W4A16_VARIANT_BYTEWISE 5 /* misaligned-base fallback */
#define CUDALM_W4A16_VARIANT_SPLIT 6    /* M <= 32, units of a tile on separate waves */
#define CUDALM_W4A16_VARIANT_SWIGLU 7   /* kernel_regs only: the fused SwiGLU kernel */
#define CUDALM_W4A16_VARIANT_PREFILL32 8 /* 32x32 MFMA GEMM, 32 x 256 per workgroup */
int cudalm_w4a16_gemv_bf16_variant(const uint8_t* weight, const uint16_t* scale,
                                   const uint16_t* x, uint16_t* y, int N, int K,
                                   int M, int variant, hipStream_t stream);
int cudalm_w4a16_gemv_bf16_prepacked_variant(const void* packed,
                                             const uint16_t* x, uint16_t* y,
                                             int N, int K, int M, int variant,
                                             hipStream_t stream);

/* VGPR + AGPR count of a variant's kernel, -1 if unavailable (AUTO and
 * STREAM: the M = 1 stream kernel; PREFILL: the 16x16 unit GEMM of 128 x 32
 * tiles; PREFILL32: the 32x32 GEMM at K = 1024, whose groups are split over
 * two wave sets). Replaces
 * int4_gemv_bf16_rowtile4_regs (int4_gemv_bf16.h:52) and
 * batch_int4_gemv_bf16_rowtile4_regs (batch_decode.h:67). */
int cudalm_w4a16_kernel_regs(int variant);

#ifdef __cplusplus
}
#endif

#endif
