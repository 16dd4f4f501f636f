// W4A16 device helpers shared by the engine's kernel files (gfx950): the
// weight-layout constants, the exact nibble -> bf16 decode, the activation
// pair order and the MFMA offset chain that cancels the decode's 1.5 bias.
#ifndef CUDALM_W4A16_DEVICE_H
#define CUDALM_W4A16_DEVICE_H

#include "hip_common.h"

namespace cudalm_hip {

constexpr int kGroup = 128;     // quantization group (k)
constexpr int kTileRows = 16;   // weight rows per MFMA tile
constexpr int kUnit = 8;        // groups per streamed unit
constexpr uint32_t kNegOffsetPair = 0xBFC0BFC0u;  // bf16 -1.5 in both halves

__host__ __device__ constexpr int packed_scale_pitch(int G) { return 16 * ((G + 7) / 8); }
__host__ __device__ constexpr size_t packed_tile_bytes(int G) {
  return static_cast<size_t>(G) * 1024 + 16 * static_cast<size_t>(packed_scale_pitch(G));
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// 8 nibbles (k = 0..7 of a block, nibble k at bits 4k) -> 4 bf16 pairs
// (k, k+4), each element 1.5 + q/16. ROT: the dword is the prepacked form,
// rotated left by 3 at load time, so pair 0 is already in place (one
// v_bitop3) and pairs 1..3 need one v_alignbit each: 7 VALU ops instead of 8.
__device__ __forceinline__ uint32_t rotr(uint32_t w, int s) {
  return __builtin_amdgcn_alignbit(w, w, s);
}

template <bool ROT = false>
__device__ __forceinline__ u32x4_t decode_nibbles(uint32_t w) {
  u32x4_t a;
  if constexpr (ROT) {
    a[0] = (w & 0x00780078u) ^ 0x3FC03FC0u;
    a[1] = (rotr(w, 4) & 0x00780078u) ^ 0x3FC03FC0u;
    a[2] = (rotr(w, 8) & 0x00780078u) ^ 0x3FC03FC0u;
    a[3] = (rotr(w, 12) & 0x00780078u) ^ 0x3FC03FC0u;
  } else {
    a[0] = ((w << 3) & 0x00780078u) ^ 0x3FC03FC0u;
    a[1] = ((w >> 1) & 0x00780078u) ^ 0x3FC03FC0u;
    a[2] = ((w >> 5) & 0x00780078u) ^ 0x3FC03FC0u;
    a[3] = ((w >> 9) & 0x00780078u) ^ 0x3FC03FC0u;
  }
  return a;
}

// Prepacked form of a file dword of 8 nibbles (see decode_nibbles<true>).
__host__ __device__ __forceinline__ uint32_t prepack_dword(uint32_t w) {
  return (w << 3) | (w >> 29);
}

// Natural bf16 order [x0x1 x2x3 x4x5 x6x7] -> pair order [x0x4 x1x5 x2x6 x3x7].
__device__ __forceinline__ u32x4_t pair_order(u32x4_t v) {
  u32x4_t p;
  // v_perm_b32 byte select over (hi:lo) = (v[2]:v[0]) and (v[3]:v[1]):
  // p0 = lo16(v0) | lo16(v2) << 16, p1 = hi16(v0) | hi16(v2) << 16, ...
  p[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
  p[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
  p[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
  p[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
  return p;
}

// -1.5 * (sum over the group of this lane-set's activation rows), as a 16x16
// accumulator tile (all columns equal).
__device__ __forceinline__ f32x4_t group_offset(const u32x4_t (&xa)[4]) {
  const u32x4_t neg = {kNegOffsetPair, kNegOffsetPair, kNegOffsetPair, kNegOffsetPair};
  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t c = mfma16(xa[0], neg, zero);
  c = mfma16(xa[1], neg, c);
  c = mfma16(xa[2], neg, c);
  c = mfma16(xa[3], neg, c);
  return c;
}

// The reference's own loop for one output (tests/cuda/test_int4_gemv_bf16.cpp:
// 54-69; the fp16 twin, tests/cuda/test_int4_gemv.cpp:49-63): fp32, k
// ascending, each term (q * f32(s)) * f32(x). The kernels call it only for
// an output whose fast sum is NaN. That sum cancels the decode's 1.5 bias
// with a second chain over -1.5 * x, so an infinite activation turns into
// Inf - Inf there, where the reference gives +-Inf when every infinite term
// has one sign (and NaN otherwise, or for a NaN activation, or a zero weight
// or scale times an infinity); overflowing finite sums are the same case.
// Recomputing those outputs in the reference's order gives the reference's
// result. W is the projection's weights (file layout [N, K/2], or prepacked:
// tile-major, dwords rotated left by 3), S its fp16 scales (file layout
// only), xrow the activation row (bf16, or fp16 when F16), read with
// device-coherent loads when XCOH (x written by another workgroup of the
// same launch).
template <bool PACKED, bool F16 = false, bool XCOH = false>
__device__ __forceinline__ float w4a16_ref_dot(const uint8_t* W, const uint16_t* S, int K, int n,
                                            const uint16_t* xrow) {
  const int G = K >> 7;
  const uint8_t* tile = W + static_cast<size_t>(n >> 4) * packed_tile_bytes(G);
  const int i = n & 15;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    const int g = k >> 7;
    int nib;
    float s;
    if constexpr (PACKED) {
      const int kk = k & 127;
      const uint32_t w = *reinterpret_cast<const uint32_t*>(
          tile + static_cast<size_t>(g) * 1024 + 16 * (16 * (kk >> 5) + i) + 4 * ((kk >> 3) & 3));
      nib = static_cast<int>((rotr(w, 3) >> (4 * (kk & 7))) & 15u);
      s = half_bits_to_f32(*reinterpret_cast<const uint16_t*>(
          tile + static_cast<size_t>(G) * 1024 + i * packed_scale_pitch(G) + 2 * g));
    } else {
      const uint8_t b = W[static_cast<size_t>(n) * (K >> 1) + (k >> 1)];
      nib = (k & 1) ? (b >> 4) : (b & 15);
      s = half_bits_to_f32(S[static_cast<size_t>(n) * G + g]);
    }
    const float q = static_cast<float>((nib ^ 8) - 8);
    const uint32_t xb =
        XCOH ? __hip_atomic_load(xrow + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : xrow[k];
    const float x = F16 ? half_bits_to_f32(xb) : bf16_lo(xb);
    acc += (q * s) * x;
  }
  return acc;
}

// y = bf16( f32(bf16(g / (1 + exp(-g)))) * u ) on bf16 inputs g, u: SiLU in
// fp32, rounded to bf16 first, then the product rounded once
// (include/cudalm/kernels/qwen35_kernels.h:146-152).
// silu_mul_bits(g, u) == mul_bits(silu_bits(g), u): the two roundings as
// separate steps, for callers that have g before u.
__device__ __forceinline__ uint32_t silu_bits(uint32_t g_bits) {
  const float g = bf16_lo(g_bits);
  return f32_to_bf16_rne(g / (1.0f + expf(-g)));
}
__device__ __forceinline__ uint32_t mul_bits(uint32_t s_bits, uint32_t u_bits) {
  return f32_to_bf16_rne(bf16_lo(s_bits) * bf16_lo(u_bits));
}
__device__ __forceinline__ uint32_t silu_mul_bits(uint32_t g_bits, uint32_t u_bits) {
  return mul_bits(silu_bits(g_bits), u_bits);
}

// Prefill-chunk GEMM on 32 x 32 MFMA tiles (w4a16_gemm.hip): 32 activation
// rows x 256 weight rows per 8-wave workgroup, any M, N and K % 128 == 0.
template <bool PACKED>
int launch_prefill32(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                     int K, int M, hipStream_t stream);

// Waves per wave set of the K = 1024 split 32x32 kernel for an N x 1024 x M
// GEMM on `cus` CUs, 0 when the unit GEMM serves the shape better.
int prefill_split_waves(int N, int M, int cus, bool packed);

// Registers per lane of that kernel at K = 1024 (prepacked instance).
int prefill32_regs();

}  // namespace cudalm_hip

#endif
