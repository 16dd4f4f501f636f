// C entry points over the reference's header-only stage comparison code
// (include/cudalm/stage_compare.h:28-137), compiled in place from the
// reference tree by oracle/build_oracle.py. Test infrastructure only.
#include <cstddef>
#include <cstdint>
#include <cstring>

#include "cudalm/stage_compare.h"

extern "C" {

float ref_fp16_bits_to_f32(std::uint16_t h) { return cudalm::fp16_bits_to_f32(h); }

// Bit pattern of the decoded float (no float return-path NaN quieting).
std::uint32_t ref_fp16_bits_to_f32_bits(std::uint16_t h) {
  const float f = cudalm::fp16_bits_to_f32(h);
  std::uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
float ref_bf16_bits_to_f32(std::uint16_t h) { return cudalm::bf16_bits_to_f32(h); }

// Returns 1 when every element passes |a - r| <= atol + rtol * |r|.
int ref_compare_bf16_stages(const std::uint16_t* ref, const std::uint16_t* act, std::size_t n,
                            double atol, double rtol, double* max_abs_err,
                            std::size_t* max_abs_idx) {
  const cudalm::StageCompareResult r = cudalm::compare_bf16_stages(ref, act, n, atol, rtol);
  if (max_abs_err) *max_abs_err = r.max_abs_err;
  if (max_abs_idx) *max_abs_idx = r.max_abs_idx;
  return r.ok ? 1 : 0;
}

// Returns 1 when every element passes |a - r| <= atol + rtol * |r| (fp16).
int ref_compare_fp16_stages(const std::uint16_t* ref, const std::uint16_t* act, std::size_t n,
                            double atol, double rtol, double* max_abs_err,
                            std::size_t* max_abs_idx) {
  const cudalm::StageCompareResult r = cudalm::compare_fp16_stages(ref, act, n, atol, rtol);
  if (max_abs_err) *max_abs_err = r.max_abs_err;
  if (max_abs_idx) *max_abs_idx = r.max_abs_idx;
  return r.ok ? 1 : 0;
}

}
