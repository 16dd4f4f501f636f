// Host side of the W4A16 engine: the C++ entry points with the reference's
// names (fatal-abort error model) and the host-memory repack.
//
// Reference interfaces replaced here:
//   cudalm::int4_gemv_bf16                include/cudalm/kernels/int4_gemv_bf16.h:46-52
//   cudalm::kernels::batch_int4_gemv_bf16 include/cudalm/kernels/batch_decode.h:61-67
//   cudalm::int4_gemv                     include/cudalm/kernels/int4_gemv.h:22-40
//   cudalm::bf16_gemv                     include/cudalm/kernels/bf16_gemv.h:37-38
//   cudalm::kernels::batch_bf16_gemv      include/cudalm/kernels/batch_decode.h:77-79
//   cudalm::kernels::qwen35_silu_mul_bf16 include/cudalm/kernels/qwen35_kernels.h:146-155
//   CUDALM_PRECONDITION / CUDA_CHECK_LAUNCH (abort)  include/cudalm/cuda_check.h:38-63

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "cudalm/kernels/batch_decode.h"
#include "cudalm/kernels/bf16_gemv.h"
#include "cudalm/kernels/int4_gemv.h"
#include "cudalm/kernels/int4_gemv_bf16.h"
#include "cudalm/kernels/swiglu.h"
#include "cudalm/w4a16_linear.h"
#include "cudalm_bf16_gemv.h"
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
std::uint16_t* bits(__half* p) { return reinterpret_cast<std::uint16_t*>(p); }

}  // namespace

void int4_gemv(const std::uint8_t* weight, const __half* scales, const __half* x, __half* y,
               int N, int K, hipStream_t stream) {
  W4A16_CHECK("int4_gemv",
              cudalm_w4a16_gemv_f16(weight, bits(scales), bits(x), bits(y), N, K, 1, stream));
}

void bf16_gemv(const __hip_bfloat16* weight, const __hip_bfloat16* x, __hip_bfloat16* y, int N,
               int K, hipStream_t stream) {
  W4A16_CHECK("bf16_gemv", cudalm_bf16_gemv(bits(weight), bits(x), bits(y), N, K, 1, stream));
}

void int4_gemv_bf16(const std::uint8_t* weight, const __half* scales, const __hip_bfloat16* x,
                    __hip_bfloat16* y, int N, int K, hipStream_t stream) {
  W4A16_CHECK("int4_gemv_bf16",
              cudalm_w4a16_gemv_bf16(weight, bits(scales), bits(x), bits(y), N, K, 1, stream));
}

int int4_gemv_bf16_rowtile4_regs() { return cudalm_w4a16_kernel_regs(CUDALM_W4A16_VARIANT_STREAM); }

namespace kernels {

void batch_bf16_gemv(const __hip_bfloat16* weight, const __hip_bfloat16* x, __hip_bfloat16* y,
                     int N, int K, int B, hipStream_t stream) {
  W4A16_CHECK("batch_bf16_gemv",
              cudalm_bf16_gemv(bits(weight), bits(x), bits(y), N, K, B, stream));
}

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

void w4a16_swiglu_forward_bf16(const PackedW4A16Linear& gate, const PackedW4A16Linear& up,
                               const __hip_bfloat16* x, __hip_bfloat16* y, int M,
                               hipStream_t stream) {
  W4A16_CHECK("w4a16_swiglu_forward_bf16",
              (gate.N != up.N || gate.K != up.K)
                  ? CUDALM_W4A16_EINVAL
                  : cudalm_w4a16_swiglu_bf16(gate.packed, nullptr, up.packed, nullptr, bits(x),
                                             bits(y), gate.N, gate.K, M, 1, stream));
}

namespace kernels {

void qwen35_silu_mul_bf16(const __hip_bfloat16* gate, const __hip_bfloat16* up,
                          __hip_bfloat16* y, std::size_t n, hipStream_t stream) {
  W4A16_CHECK("qwen35_silu_mul_bf16", cudalm_silu_mul_bf16(bits(gate), bits(up), bits(y), n, stream));
}

}  // namespace kernels

}  // namespace cudalm

extern "C" int cudalm_w4a16_repack_host(const uint8_t* weight, const uint16_t* scale,
                                        void* packed, int N, int K) {
  if (N < 1 || K <= 0 || K % CUDALM_W4A16_GROUP != 0) return CUDALM_W4A16_EINVAL;
  if (!weight || !scale || !packed) return CUDALM_W4A16_ENULL;
  // Layout (the kernels' prepacked form): per 16-row tile, G groups of
  // 1024 weight bytes (lane l = 16a + i: row i, bytes [16a, 16a+16) of the
  // group, each dword rotated left by 3 bits), then 16 rows of scales with a pitch of 16 * ceil(G/8) bytes.
  const int G = K / CUDALM_W4A16_GROUP;
  const int SP = 16 * ((G + 7) / 8);
  const std::size_t tile_bytes = static_cast<std::size_t>(G) * 1024 + 16 * static_cast<std::size_t>(SP);
  const int ntiles = (N + 15) / 16;
  std::uint8_t* out = static_cast<std::uint8_t*>(packed);
  for (int rt = 0; rt < ntiles; ++rt) {
    std::uint8_t* tile = out + static_cast<std::size_t>(rt) * tile_bytes;
    for (int g = 0; g < G; ++g) {
      for (int l = 0; l < 64; ++l) {
        const int n = rt * 16 + (l & 15);
        const int a = l >> 4;
        std::uint8_t* dst = tile + static_cast<std::size_t>(g) * 1024 + 16 * l;
        if (n < N) {
          // each little-endian dword of 8 nibbles is stored rotated left by 3
          const std::uint8_t* src = weight + static_cast<std::size_t>(n) * (K / 2) + g * 64 + a * 16;
          for (int q = 0; q < 4; ++q) {
            std::uint32_t w;
            std::memcpy(&w, src + 4 * q, 4);
            w = (w << 3) | (w >> 29);
            std::memcpy(dst + 4 * q, &w, 4);
          }
        } else {
          std::memset(dst, 0, 16);
        }
      }
    }
    std::uint8_t* srows = tile + static_cast<std::size_t>(G) * 1024;
    std::memset(srows, 0, 16 * static_cast<std::size_t>(SP));
    for (int r = 0; r < 16; ++r) {
      const int n = rt * 16 + r;
      if (n < N)
        std::memcpy(srows + static_cast<std::size_t>(r) * SP,
                    scale + static_cast<std::size_t>(n) * G, 2 * static_cast<std::size_t>(G));
    }
  }
  return CUDALM_W4A16_OK;
}
