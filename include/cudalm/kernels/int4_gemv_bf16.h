// MI355X W4A16 GEMV, C++ entry point with the reference's name and argument
// order (reference: include/cudalm/kernels/int4_gemv_bf16.h:29-52).
//
//   y[n] = bf16_rne( sum_k unpack(weight)[n,k] * f32(scales[n,k/128]) * f32(x[k]) )
//
//   weight : packed int4 [N, K/2] uint8 row-major; low nibble = k = 2b,
//            high nibble = k = 2b+1 (4-bit two's complement)
//   scales : fp16 [N, K/128] row-major
//   x      : bf16 [K];  y : bf16 [N]
//
// Preconditions N >= 1 and K % 128 == 0 abort with a diagnostic when
// violated, as in the reference (cuda_check.h:53-63). Misaligned weight or
// x bases are served by a byte-wise kernel; legal inputs are never rejected.
// The call is asynchronous on `stream` and allocates nothing.
#pragma once

#include <cstdint>

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

namespace cudalm {

void int4_gemv_bf16(const std::uint8_t* weight, const __half* scales,
                    const __hip_bfloat16* x, __hip_bfloat16* y, int N, int K,
                    hipStream_t stream);

// Register count (VGPR + AGPR) of the M = 1 kernel; -1 if unavailable.
int int4_gemv_bf16_rowtile4_regs();

}  // namespace cudalm
