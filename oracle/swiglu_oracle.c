/*
 * SwiGLU element-wise stage, CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates qwen35_silu_mul_kernel (src/kernels/qwen35_kernels.cu:458-476;
 * contract include/cudalm/kernels/qwen35_kernels.h:146-152):
 *   s = bf16_rne( g / (1 + expf(-g)) ),  y = bf16_rne( f32(s) * f32(u) )
 * with g, u the bf16 inputs widened to fp32. Only tests/ and bench.py's
 * cpu_baseline leg load it, as the checker.
 *
 * Pinning status: orc_silu_bf16 against the correctly rounded bf16 of the
 * fp64 SiLU over all 65536 bf16 inputs (all but near-tie cases equal);
 * orc_silu_mul_bf16 against the exact fp64 product rounded once.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include "w4a16_oracle.h"

uint16_t orc_silu_bf16(uint16_t g_bits) {
  const float g = orc_bf16_to_f32(g_bits);
  const float e = expf(-g);
  const float d = 1.0f + e;
  return orc_f32_to_bf16_rne(g / d);
}

void orc_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float s = orc_bf16_to_f32(orc_silu_bf16(gate[i]));
    const float p = s * orc_bf16_to_f32(up[i]);
    y[i] = orc_f32_to_bf16_rne(p);
  }
}
