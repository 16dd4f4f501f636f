// Host side of the W4A16 engine: the C++ entry points with the reference's
// names (fatal-abort error model) and the host-memory repack.
//
// Reference interfaces replaced here:
//   cudalm::int4_gemv_bf16                include/cudalm/kernels/int4_gemv_bf16.h:46-52
//   cudalm::kernels::batch_int4_gemv_bf16 include/cudalm/kernels/batch_decode.h:61-67
//   CUDALM_PRECONDITION / CUDA_CHECK_LAUNCH (abort)  include/cudalm/cuda_check.h:38-63

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "cudalm/kernels/batch_decode.h"
#include "cudalm/kernels/int4_gemv_bf16.h"
#include "cudalm/w4a16_linear.h"
#include "cudalm_w4a16.h"

namespace cudalm {
namespace {

[[noreturn]] void w4a16_fatal(const char* entry, int code, const char* file, int line) {
  std::fprintf(stderr,
               "[cudalm] %s: %s\n"
               "  code       : %d\n"
               "  file       : %s:%d\n",
               entry, cudalm_w4a16_strerror(code), code, file, line);
  std::abort();
}

#define W4A16_CHECK(entry, call)                                       \
  do {                                                                 \
    const int w4a16_rc__ = (call);                                     \
    if (w4a16_rc__ != CUDALM_W4A16_OK) w4a16_fatal(entry, w4a16_rc__, __FILE__, __LINE__); \
  } while (0)

const std::uint16_t* bits(const __half* p) { return reinterpret_cast<const std::uint16_t*>(p); }
const std::uint16_t* bits(const __hip_bfloat16* p) {
  return reinterpret_cast<const std::uint16_t*>(p);
}
std::uint16_t* bits(__hip_bfloat16* p) { return reinterpret_cast<std::uint16_t*>(p); }

}  // namespace

void int4_gemv_bf16(const std::uint8_t* weight, const __half* scales, const __hip_bfloat16* x,
                    __hip_bfloat16* y, int N, int K, hipStream_t stream) {
  W4A16_CHECK("int4_gemv_bf16",
              cudalm_w4a16_gemv_bf16(weight, bits(scales), bits(x), bits(y), N, K, 1, stream));
}

int int4_gemv_bf16_rowtile4_regs() { return cudalm_w4a16_kernel_regs(CUDALM_W4A16_VARIANT_STREAM); }

namespace kernels {

void batch_int4_gemv_bf16(const std::uint8_t* weight, const __half* scale,
                          const __hip_bfloat16* x, __hip_bfloat16* y, int N, int K, int B,
                          hipStream_t stream) {
  W4A16_CHECK("batch_int4_gemv_bf16",
              cudalm_w4a16_gemv_bf16(weight, bits(scale), bits(x), bits(y), N, K, B, stream));
}

int batch_int4_gemv_bf16_rowtile4_regs() {
  return cudalm_w4a16_kernel_regs(CUDALM_W4A16_VARIANT_TILE16);
}

}  // namespace kernels

std::size_t packed_w4a16_bytes(int N, int K) { return cudalm_w4a16_packed_bytes(N, K); }

PackedW4A16Linear repack_w4a16(const W4A16LinearView& lin, void* dst, hipStream_t stream) {
  W4A16_CHECK("repack_w4a16",
              cudalm_w4a16_repack(lin.weight, bits(lin.scale), dst, lin.N, lin.K, stream));
  PackedW4A16Linear p;
  p.packed = dst;
  p.N = lin.N;
  p.K = lin.K;
  return p;
}

void repack_w4a16_host(const std::uint8_t* weight, const std::uint16_t* scale, int N, int K,
                       void* dst_host) {
  W4A16_CHECK("repack_w4a16_host", cudalm_w4a16_repack_host(weight, scale, dst_host, N, K));
}

void w4a16_forward_bf16(const PackedW4A16Linear& lin, const __hip_bfloat16* x, __hip_bfloat16* y,
                        int M, hipStream_t stream) {
  W4A16_CHECK("w4a16_forward_bf16",
              cudalm_w4a16_gemv_bf16_prepacked(lin.packed, bits(x), bits(y), lin.N, lin.K, M,
                                               stream));
}

}  // namespace cudalm

extern "C" int cudalm_w4a16_repack_host(const uint8_t* weight, const uint16_t* scale,
                                        void* packed, int N, int K) {
  if (N < 1 || K <= 0 || K % CUDALM_W4A16_GROUP != 0) return CUDALM_W4A16_EINVAL;
  if (!weight || !scale || !packed) return CUDALM_W4A16_ENULL;
  const int G = K / CUDALM_W4A16_GROUP;
  const int ntiles = (N + 15) / 16;
  std::uint8_t* out = static_cast<std::uint8_t*>(packed);
  const std::uint8_t* sb = reinterpret_cast<const std::uint8_t*>(scale);
  for (int rt = 0; rt < ntiles; ++rt) {
    for (int g = 0; g < G; ++g) {
      std::uint8_t* blk = out + (static_cast<std::size_t>(rt) * G + g) * 1056;
      for (int l = 0; l < 64; ++l) {
        const int n = rt * 16 + (l & 15);
        const int a = l >> 4;
        if (n < N)
          std::memcpy(blk + 16 * l, weight + static_cast<std::size_t>(n) * (K / 2) + g * 64 + a * 16,
                      16);
        else
          std::memset(blk + 16 * l, 0, 16);
      }
      for (int r = 0; r < 16; ++r) {
        const int n = rt * 16 + r;
        if (n < N)
          std::memcpy(blk + 1024 + 2 * r, sb + (static_cast<std::size_t>(n) * G + g) * 2, 2);
        else
          std::memset(blk + 1024 + 2 * r, 0, 2);
      }
    }
  }
  return CUDALM_W4A16_OK;
}
