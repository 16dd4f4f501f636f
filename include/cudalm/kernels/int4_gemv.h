// MI355X W4A16 GEMV with fp16 activations, C++ entry point with the
// reference's name and argument order (reference: include/cudalm/kernels/
// int4_gemv.h:22-40).
//
// y[n] = sum_k unpack(weight)[n,k] * scales[n, k/128] * x[k], fp32
// accumulation, one fp16 RNE store. weight packed int4 [N, K/2], scales
// fp16 [N, K/128], x fp16 [K], y fp16 [N]. Preconditions N >= 1,
// K % 128 == 0 abort when violated; misaligned bases are served (byte-wise
// kernel), as the reference requires. Asynchronous on `stream`.
#pragma once

#include <cstdint>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

namespace cudalm {

void int4_gemv(const std::uint8_t* weight, const __half* scales, const __half* x, __half* y,
               int N, int K, hipStream_t stream);

}  // namespace cudalm
