// MI355X bf16 GEMV (tied LM head), C++ entry point with the reference's
// name and argument order (reference: include/cudalm/kernels/bf16_gemv.h:
// 19-38).
//
// y[n] = sum_k W[n,k] * x[k], fp32 accumulation, one bf16 RNE store.
// weight bf16 [N, K] row-major, x bf16 [K], y bf16 [N]. Any N >= 1, K >= 1
// and any (2-byte aligned) bases: K % 8 == 0 with 16 B aligned bases takes
// the matrix-core kernel, anything else the element-wise kernel. A
// violated precondition aborts, as CUDALM_PRECONDITION does. Asynchronous
// on `stream`.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

namespace cudalm {

void bf16_gemv(const __hip_bfloat16* weight, const __hip_bfloat16* x, __hip_bfloat16* y, int N,
               int K, hipStream_t stream);

}  // namespace cudalm
