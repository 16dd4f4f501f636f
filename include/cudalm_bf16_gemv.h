/*
 * cudalm_bf16_gemv -- C ABI of the MI355X (gfx950) bf16 GEMV: the tied
 * LM head (logits = embed_tokens.weight x final hidden).
 *
 * Arithmetic contract (the reference's, include/cudalm/kernels/
 * bf16_gemv.h:19-38 and batch_decode.h:69-79):
 *
 *   y[m, n] = bf16_rne( sum_k f32(weight[n, k]) * f32(x[m, k]) )
 *
 *   weight : bf16 bit patterns [N, K], row-major.
 *   x      : bf16 bit patterns [M, K], row-major (M activation rows).
 *   y      : bf16 bit patterns [M, N], row-major.
 *
 * fp32 accumulation, one bf16 round-to-nearest-even per output. Results are
 * within 2 bf16 ulp of the exact sum plus a floor for outputs that cancel
 * (the tests state it). Row m of a batched call is bit-identical to a
 * single-row call on row m.
 *
 * Any N >= 1, K >= 1, M >= 1 and any 2-byte-aligned bases are accepted:
 * K % 8 == 0 with 16 B aligned weight and x takes the matrix-core stream
 * kernel, everything else an element-wise kernel (the reference's policy,
 * bf16_gemv.h:27-33). Ownership, threading and the error model are those
 * of cudalm_w4a16.h (same CUDALM_W4A16_E* codes; EINVAL here means N, K or
 * M < 1, EALIGN a base that is not 2-byte aligned).
 */
#ifndef CUDALM_BF16_GEMV_H
#define CUDALM_BF16_GEMV_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "cudalm_w4a16.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CUDALM_BF16_VARIANT_AUTO 0
#define CUDALM_BF16_VARIANT_STREAM 1 /* MFMA stream kernel (K % 8 == 0, 16 B bases) */
#define CUDALM_BF16_VARIANT_SCALAR 2 /* element-wise kernel, any layout */

/* y[M, N] = weight[N, K] applied to x[M, K]. Replaces bf16_gemv (M == 1;
 * include/cudalm/kernels/bf16_gemv.h:37-38) and kernels::batch_bf16_gemv
 * (M == B; include/cudalm/kernels/batch_decode.h:77-79). */
int cudalm_bf16_gemv(const uint16_t* weight, const uint16_t* x, uint16_t* y,
                     int N, int K, int M, hipStream_t stream);

/* Same, forcing one kernel (tests, measurement). CUDALM_W4A16_EVARIANT if
 * the kernel cannot serve the call. */
int cudalm_bf16_gemv_variant(const uint16_t* weight, const uint16_t* x,
                             uint16_t* y, int N, int K, int M, int variant,
                             hipStream_t stream);

/* Registers (VGPR + AGPR) of a variant's kernel; -1 if unavailable. */
int cudalm_bf16_gemv_kernel_regs(int variant);

/* Load-time tile repack of a bf16 weight (no counterpart in the reference;
 * it hooks where the tied embedding is uploaded, the upload lambda of
 * src/runtime/weight_loader_v2.cpp:435-441, like cudalm_w4a16_repack).
 * The packed copy is tile-major: for each 16-row tile and each 256-k unit,
 * eight 1 KB slabs, slab j holding at byte 16 l the 16 bytes MFMA lane l
 * reads at step j (row 16 t + l % 16, k = 256 u + 32 j + 8 (l / 16)), so
 * every wave-wide load of the GEMV reads 1 KB contiguous. The row-major
 * original stays valid (the embedding lookup reads it); the copy is a
 * second N*K*2 bytes. Requires N % 16 == 0, K % 256 == 0 and 16-byte
 * aligned bases (CUDALM_W4A16_EINVAL / EALIGN otherwise). The packed size
 * is N * K * 2 bytes; cudalm_bf16_packed_bytes returns 0 for a shape the
 * packed path does not take. */
size_t cudalm_bf16_packed_bytes(int N, int K);
int cudalm_bf16_repack(const uint16_t* weight, void* packed, int N, int K,
                       hipStream_t stream);

/* cudalm_bf16_gemv on the packed copy: the same kernel and the same result
 * bits, reading 1 KB contiguous per wave load. N % 16 == 0, K % 256 == 0,
 * 16-byte aligned packed and x bases, and x rows that fit the LDS
 * (CUDALM_W4A16_EVARIANT otherwise). */
int cudalm_bf16_gemv_prepacked(const void* packed, const uint16_t* x, uint16_t* y,
                               int N, int K, int M, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
