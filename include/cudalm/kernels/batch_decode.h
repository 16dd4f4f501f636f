// MI355X W4A16 batched GEMV, C++ entry point with the reference's name and
// argument order (reference: include/cudalm/kernels/batch_decode.h:48-67).
//
// y_b = W * x_b for b = 0..B-1, x bf16 [B, K], y bf16 [B, N]. Row b of the
// output is bit-identical to int4_gemv_bf16 on x_b alone (the reference's
// row-parity contract, tests/cuda/test_qwen35_batch_kernels.cpp:86-125).
// Any B >= 1 is accepted: B <= 32 runs the small-M decode kernels, larger B
// (prefill chunks) the MFMA tile kernel. Preconditions N >= 1, B >= 1,
// K % 128 == 0 abort when violated. Asynchronous on `stream`.
#pragma once

#include <cstdint>

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

namespace cudalm {
namespace kernels {

void batch_int4_gemv_bf16(const std::uint8_t* weight, const __half* scale,
                          const __hip_bfloat16* x, __hip_bfloat16* y, int N,
                          int K, int B, hipStream_t stream);

// Register count (VGPR + AGPR) of the small-M kernel; -1 if unavailable.
int batch_int4_gemv_bf16_rowtile4_regs();

// bf16 GEMV (tied LM head), B rows: y_b = W * x_b, x bf16 [B, K], y bf16
// [B, N] (reference: include/cudalm/kernels/batch_decode.h:69-79). The
// weight is streamed once for up to 32 rows; row b is bit-identical to
// bf16_gemv on x_b alone. Any K >= 1 and 2-byte aligned bases.
void batch_bf16_gemv(const __hip_bfloat16* weight, const __hip_bfloat16* x,
                     __hip_bfloat16* y, int N, int K, int B, hipStream_t stream);

}  // namespace kernels
}  // namespace cudalm
