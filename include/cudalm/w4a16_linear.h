// W4A16 projection handles for the model runtime: the file-layout view the
// reference's loader fills (reference: include/cudalm/weight_loader.h:57-63,
// src/runtime/weight_loader_v2.cpp:435-441,479-482) and the load-time
// repacked form the MI355X kernels stream fastest.
#pragma once

#include <cstddef>
#include <cstdint>

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

namespace cudalm {

// File layout: weight [N, K/2] packed int4, scale [N, K/128] fp16.
struct W4A16LinearView {
  const std::uint8_t* weight = nullptr;
  const __half* scale = nullptr;
  int N = 0;
  int K = 0;
};

// Repacked layout: ceil(N/16) tiles of (K/128) * 1024 + 256 * ceil(K/1024) bytes.
struct PackedW4A16Linear {
  void* packed = nullptr;  // device buffer owned by the caller
  int N = 0;
  int K = 0;
};

// Bytes of the repacked form; 0 for an invalid shape.
std::size_t packed_w4a16_bytes(int N, int K);

// Repack a device-resident file-layout projection into `dst` (caller-owned,
// packed_w4a16_bytes(N, K) bytes, 16 B aligned). Aborts on a contract
// violation, like the reference's CUDALM_PRECONDITION. Stream-ordered.
PackedW4A16Linear repack_w4a16(const W4A16LinearView& lin, void* dst,
                               hipStream_t stream);

// Repack host-resident file bytes into a host staging buffer, for a loader
// that uploads once after the repack. Aborts on a contract violation.
void repack_w4a16_host(const std::uint8_t* weight, const std::uint16_t* scale,
                       int N, int K, void* dst_host);

// y[M, N] = lin(x[M, K]); bit-identical to the file-layout entry points.
void w4a16_forward_bf16(const PackedW4A16Linear& lin, const __hip_bfloat16* x,
                        __hip_bfloat16* y, int M, hipStream_t stream);

// y[M, N] = silu(gate(x)) * up(x) with the reference's roundings (gate and
// up outputs as bf16, SiLU rounded to bf16, then the product), one launch;
// equal to w4a16_forward_bf16 on each projection followed by
// kernels::qwen35_silu_mul_bf16. gate and up must share N and K.
void w4a16_swiglu_forward_bf16(const PackedW4A16Linear& gate, const PackedW4A16Linear& up,
                               const __hip_bfloat16* x, __hip_bfloat16* y, int M,
                               hipStream_t stream);

}  // namespace cudalm
