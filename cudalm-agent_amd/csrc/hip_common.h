// Device and launch helpers shared by the engine's kernel files (gfx950).
#ifndef CUDALM_HIP_COMMON_H
#define CUDALM_HIP_COMMON_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <stdlib.h>

#include <atomic>

#include "cudalm_w4a16.h"

namespace cudalm_hip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr size_t kLdsMax = 160 * 1024;  // LDS per CU (and per workgroup) on gfx950

// Wave index inside the workgroup, as a wave-uniform (scalar) value.
// Orders one wave's LDS writes before its later LDS reads (and those reads
// before later writes) when lanes exchange data through LDS: the LDS unit
// serves a wave's operations in order, so only the compiler needs fencing.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) {
  return __builtin_bit_cast(float, v & 0xFFFF0000u);
}

// fp32 -> bf16, round to nearest even; a NaN becomes the quiet NaN
// (x >> 16) | 0x40. One v_cvt_pk_bf16_f32: over all 2^32 fp32 inputs it
// gives the same 16 bits as the integer form
//   NaN ? (x >> 16) | 0x40 : (x + 0x7FFF + ((x >> 16) & 1)) >> 16
// (checked exhaustively on gfx950), which is what the oracle computes.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// D = A (16 rows x 32 k) * B (32 k x 16 cols) + C, bf16 in, fp32 accumulate.
// Lane l = 16a + i: A row i / B column i, k = 8a .. 8a+7; D rows 4a..4a+3 of column i.
__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

constexpr int kMaxDevices = 64;

inline int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  return dev;
}

// Compute units of the current device (cached per device; the cache is
// filled with relaxed atomics, every writer stores the same value).
inline int cu_count() {
  static std::atomic<int> cached[kMaxDevices];
  const int dev = current_device();
  if (dev < 0) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? CUDALM_W4A16_OK : CUDALM_W4A16_ELAUNCH;
}

// Dynamic LDS above 64 KB must be opted into, per kernel and device. The
// opt-in is remembered per host thread for up to 64 (device, kernel) pairs;
// beyond that it is simply repeated.
template <typename F>
bool allow_lds(F kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return true;
  if (bytes > kLdsMax) return false;
  struct Entry {
    const void* fn;
    int dev;
  };
  static thread_local Entry done[64] = {};
  const void* fn = reinterpret_cast<const void*>(kernel);
  const int dev = current_device();
  for (auto& d : done) {
    if (d.fn == fn && d.dev == dev) return true;
    if (d.fn == nullptr) {
      if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(kLdsMax)) != hipSuccess)
        return false;
      d = {fn, dev};
      return true;
    }
  }
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(kLdsMax)) == hipSuccess;
}

template <typename F>
int regs_of(F kernel) {
  hipFuncAttributes attr;
  if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kernel)) != hipSuccess) return -1;
  return attr.numRegs;
}

}  // namespace cudalm_hip

#endif
