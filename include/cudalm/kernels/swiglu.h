// MI355X SwiGLU element-wise stage, C++ entry point with the reference's
// name and argument order (reference: include/cudalm/kernels/
// qwen35_kernels.h:146-155).
//
// y[i] = bf16( f32(silu_bf16) * f32(up[i]) ),
// silu_bf16 = bf16( f32(gate[i]) / (1 + exp(-f32(gate[i]))) ),
// bf16 [n] buffers. Any n and 2-byte aligned bases are accepted (the
// reference requires n % 8 == 0 and 16 B aligned bases). Asynchronous on
// `stream`; a violated precondition aborts.
#pragma once

#include <cstddef>

#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

namespace cudalm {
namespace kernels {

void qwen35_silu_mul_bf16(const __hip_bfloat16* gate, const __hip_bfloat16* up,
                          __hip_bfloat16* y, std::size_t n, hipStream_t stream);

}  // namespace kernels
}  // namespace cudalm
