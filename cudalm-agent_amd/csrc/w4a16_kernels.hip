// W4A16 projection engine for MI355X (gfx950): kernels and the C-ABI launch
// layer declared in include/cudalm_w4a16.h.
//
// Contract (reference: include/cudalm/kernels/int4_gemv_bf16.h:6-9,29-37,
// src/kernels/int4_gemv_bf16.cu:75-170, src/kernels/batch_decode.cu:95-190):
//   y[m,n] = bf16_rne( sum_k q[n,k] * f32(s[n,k/128]) * f32(x[m,k]) ), fp32 acc.
//
// How the contraction maps onto CDNA4 matrix cores
// -------------------------------------------------
// Every kernel below computes 16-row x 16-column output tiles with
// v_mfma_f32_16x16x32_bf16 (A = weights, rows n; B = activations, columns m).
// One 128-wide quantization group of one 16-row tile is a 1 KB slab of
// packed weights: lane l = 16*a + i loads the 16 bytes of row i that hold
// k = 32a .. 32a+31 of the group, and each of its four dwords feeds one MFMA
// step (8 k per lane per step, 32 k per step).
//
// A weight nibble n (two's complement q) is turned into an exact bf16 by
// bit placement alone: bits 0x3F80 | ((n ^ 8) << 3) encode 1 + (q+8)/16 =
// 1.5 + q/16. Two nibbles 16 bits apart become one bf16 pair with a shift
// and one v_bitop3, so a dword of 8 nibbles costs 8 VALU ops. The constant
// 1.5 is removed per group and column:
//     sum_k q x = 16 * ( sum_k (1.5 + q/16) x  -  1.5 * sum_k x )
// and the fp16 scale is applied once per group in fp32:
//     acc = fma(s[n,g], tmp[n,m,g] - c[m,g], acc),   c[m,g] = 1.5 * sum_{k in g} x[m,k]
// with the final y = bf16_rne(16 * acc). The pair layout the bit placement
// produces is (k, k+4) for k = 0..3 of every 8-k block, so activations are
// stored in LDS in that order: [x0 x4 x1 x5 x2 x6 x3 x7].
//
// Every kernel uses the same per-element operation sequence (same MFMA
// operands, same group order, same epilogue), so one output element has the
// same bits whichever kernel, tile shape, batch size or weight layout
// produced it. The tests pin that.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "cudalm_w4a16.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kGroup = 128;          // quantization group (k)
constexpr int kTileRows = 16;        // output rows per MFMA tile
constexpr int kPackedBlock = 1056;   // prepacked bytes per (16-row tile, group)
constexpr int kPackedScaleOff = 1024;

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ __forceinline__ float bf16_lo(uint32_t v) {
  return __builtin_bit_cast(float, v << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t v) {
  return __builtin_bit_cast(float, v & 0xFFFF0000u);
}

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  const uint32_t x = __builtin_bit_cast(uint32_t, f);
  if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu)) return (x >> 16) | 0x40u;
  return (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
}

// 8 nibbles (k = 0..7 of a block, nibble k at bits 4k) -> 4 bf16 pairs
// (k, k+4), each element 1.5 + q/16.
__device__ __forceinline__ u32x4_t decode_nibbles(uint32_t w) {
  u32x4_t a;
  a[0] = ((w << 3) & 0x00780078u) ^ 0x3FC03FC0u;
  a[1] = ((w >> 1) & 0x00780078u) ^ 0x3FC03FC0u;
  a[2] = ((w >> 5) & 0x00780078u) ^ 0x3FC03FC0u;
  a[3] = ((w >> 9) & 0x00780078u) ^ 0x3FC03FC0u;
  return a;
}

// Natural bf16 order [x0x1 x2x3 x4x5 x6x7] -> pair order [x0x4 x1x5 x2x6 x3x7].
__device__ __forceinline__ u32x4_t pair_order(u32x4_t v) {
  u32x4_t p;
  p[0] = (v[0] & 0xFFFFu) | (v[2] << 16);
  p[1] = (v[0] >> 16) | (v[2] & 0xFFFF0000u);
  p[2] = (v[1] & 0xFFFFu) | (v[3] << 16);
  p[3] = (v[1] >> 16) | (v[3] & 0xFFFF0000u);
  return p;
}

__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// 1.5 * (sum of the 128 activations of one group), summed in LDS storage
// order (16 blocks ascending, pairs ascending, low element first).
__device__ __forceinline__ float group_offset(const u32x4_t* blocks) {
  float s = 0.0f;
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    const u32x4_t v = blocks[b];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s += bf16_lo(v[r]);
      s += bf16_hi(v[r]);
    }
  }
  return 1.5f * s;
}

// One group of one 16x16 tile: four MFMA steps over the lane's 16 weight
// bytes. xrow points at the lane's LDS activation row, at the group start.
__device__ __forceinline__ f32x4_t group_product(u32x4_t w, const u32x4_t* xgroup,
                                                 int a) {
  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t t = mfma16(decode_nibbles(w[0]), xgroup[4 * a + 0], zero);
  t = mfma16(decode_nibbles(w[1]), xgroup[4 * a + 1], t);
  t = mfma16(decode_nibbles(w[2]), xgroup[4 * a + 2], t);
  t = mfma16(decode_nibbles(w[3]), xgroup[4 * a + 3], t);
  return t;
}

__device__ __forceinline__ void group_epilogue(f32x4_t& acc, f32x4_t t, float c,
                                               const float (&s)[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(s[r], t[r] - c, acc[r]);
}

__device__ __forceinline__ void scales_from_u32x2(u32x2_t v, float (&s)[4]) {
  s[0] = half_bits_to_f32(v[0] & 0xFFFFu);
  s[1] = half_bits_to_f32(v[0] >> 16);
  s[2] = half_bits_to_f32(v[1] & 0xFFFFu);
  s[3] = half_bits_to_f32(v[1] >> 16);
}

// Store one lane's four outputs (rows n0..n0+3 of column m).
__device__ __forceinline__ void store_tile_column(uint16_t* __restrict__ Y, f32x4_t acc,
                                                  size_t ybase, int n0, int N) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (n0 + r < N) Y[ybase + n0 + r] = static_cast<uint16_t>(f32_to_bf16_rne(16.0f * acc[r]));
  }
}

// Stage rows [m0, m0+mrows) x k [k0, k0+kcl) of X into LDS in pair order,
// row pitch `pitch` 16-byte blocks.
__device__ __forceinline__ void stage_activations(u32x4_t* xs, int pitch,
                                                  const uint16_t* __restrict__ X,
                                                  int K, int m0, int mrows, int k0,
                                                  int kcl) {
  const int nb = kcl >> 3;
  for (int t = threadIdx.x; t < mrows * nb; t += blockDim.x) {
    const int mm = t / nb;
    const int b = t - mm * nb;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(
        X + static_cast<size_t>(m0 + mm) * K + k0 + 8 * b);
    xs[mm * pitch + b] = pair_order(v);
  }
}

__device__ __forceinline__ void stage_offsets(float* cs, int cpitch, const u32x4_t* xs,
                                              int pitch, int mrows, int ng) {
  for (int t = threadIdx.x; t < mrows * ng; t += blockDim.x) {
    const int mm = t / ng;
    const int gl = t - mm * ng;
    cs[mm * cpitch + gl] = group_offset(xs + mm * pitch + gl * 16);
  }
}

// ---------------------------------------------------------------------------
// Stream kernel: M <= 16, all of x resident in LDS, waves stream 16-row
// tiles (grid-stride), prefetching the next unit of up to 8 groups while
// the current one is computed.
// ---------------------------------------------------------------------------

constexpr int kStreamWaves = 4;
constexpr int kStreamUnit = 8;  // groups per unit

template <bool PACKED>
struct StreamUnit {
  u32x4_t w[kStreamUnit];
  u32x2_t s[kStreamUnit];  // PACKED: this lane's 4 row scales per group
  uint32_t s0, s1;         // file layout: two raw scales this lane stages
};

template <bool PACKED>
__device__ __forceinline__ void stream_load(StreamUnit<PACKED>& u,
                                            const uint8_t* __restrict__ W,
                                            const uint16_t* __restrict__ S, int N,
                                            int K, int G, int rt, int g0, int gn,
                                            int lane) {
  if constexpr (PACKED) {
    const uint8_t* base = W + (static_cast<size_t>(rt) * G + g0) * kPackedBlock;
#pragma unroll
    for (int gg = 0; gg < kStreamUnit; ++gg) {
      if (gg < gn) {
        u.w[gg] = *reinterpret_cast<const u32x4_t*>(base + gg * kPackedBlock + lane * 16);
        u.s[gg] = *reinterpret_cast<const u32x2_t*>(base + gg * kPackedBlock +
                                                    kPackedScaleOff + (lane >> 4) * 8);
      }
    }
  } else {
    const int i = lane & 15, a = lane >> 4;
    const int row = min(rt * kTileRows + i, N - 1);
    const uint8_t* wrow = W + static_cast<size_t>(row) * (K >> 1) + a * 16;
#pragma unroll
    for (int gg = 0; gg < kStreamUnit; ++gg) {
      if (gg < gn) u.w[gg] = *reinterpret_cast<const u32x4_t*>(wrow + (g0 + gg) * 64);
    }
    const int srow = min(rt * kTileRows + (lane >> 2), N - 1);
    const int gq = 2 * (lane & 3);
    const uint16_t* sp = S + static_cast<size_t>(srow) * G + g0 + gq;
    u.s0 = (gq < gn) ? sp[0] : 0u;
    u.s1 = (gq + 1 < gn) ? sp[1] : 0u;
  }
}

template <bool PACKED>
__global__ __launch_bounds__(kStreamWaves * 64) void w4a16_stream_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int K, int M) {
  extern __shared__ u32x4_t smem[];
  const int G = K >> 7;
  const int pitch = (K >> 3) + 1;
  u32x4_t* xs = smem;
  float* cs = reinterpret_cast<float*>(smem + M * pitch);
  uint16_t* ss = reinterpret_cast<uint16_t*>(cs + ((M * G + 3) & ~3));

  stage_activations(xs, pitch, X, K, 0, M, 0, K);
  __syncthreads();
  stage_offsets(cs, G, xs, pitch, M, G);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int i = lane & 15, a = lane >> 4;
  const int col = min(i, M - 1);
  const u32x4_t* xrow = xs + col * pitch;
  const float* crow = cs + col * G;
  uint16_t* wss = ss + wave * (kStreamUnit * kTileRows);

  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int U = (G + kStreamUnit - 1) / kStreamUnit;
  const int stride = gridDim.x * kStreamWaves;
  int t = blockIdx.x * kStreamWaves + wave;
  if (t >= ntiles) return;
  int u = 0;

  StreamUnit<PACKED> cur, nxt;
  stream_load<PACKED>(cur, W, S, N, K, G, t, 0, min(kStreamUnit, G), lane);
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  while (true) {
    int nt = t, nu = u + 1;
    if (nu == U) {
      nu = 0;
      nt = t + stride;
    }
    const bool has_next = nt < ntiles;
    if (has_next)
      stream_load<PACKED>(nxt, W, S, N, K, G, nt, nu * kStreamUnit,
                          min(kStreamUnit, G - nu * kStreamUnit), lane);

    const int g0 = u * kStreamUnit;
    const int gn = min(kStreamUnit, G - g0);
    if constexpr (!PACKED) {
      // transpose this unit's scales to [group][row] so each lane reads its
      // four rows of one group with one 8-byte LDS load
      const int gq = 2 * (lane & 3);
      wss[gq * kTileRows + (lane >> 2)] = static_cast<uint16_t>(cur.s0);
      wss[(gq + 1) * kTileRows + (lane >> 2)] = static_cast<uint16_t>(cur.s1);
    }
#pragma unroll
    for (int gg = 0; gg < kStreamUnit; ++gg) {
      if (gg < gn) {
        const int g = g0 + gg;
        const f32x4_t tp = group_product(cur.w[gg], xrow + g * 16, a);
        float s[4];
        if constexpr (PACKED) {
          scales_from_u32x2(cur.s[gg], s);
        } else {
          scales_from_u32x2(*reinterpret_cast<const u32x2_t*>(wss + gg * kTileRows + 4 * a), s);
        }
        group_epilogue(acc, tp, crow[g], s);
      }
    }
    if (u == U - 1) {
      if (i < M) store_tile_column(Y, acc, static_cast<size_t>(i) * N, t * kTileRows + 4 * a, N);
      acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (!has_next) break;
    cur = nxt;
    t = nt;
    u = nu;
  }
}

// ---------------------------------------------------------------------------
// Tile kernel: any M. A workgroup of WN x WM waves owns a (WN*RB*16) x
// (WM*CT*16) output tile; K is walked in chunks of GPC groups whose
// activations are staged in LDS; each wave preloads the chunk's weights.
// ---------------------------------------------------------------------------

template <int RB, int CT, int WN, int WM, int GPC, bool PACKED>
__global__ __launch_bounds__(WN * WM * 64) void w4a16_tile_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int K, int M) {
  extern __shared__ u32x4_t smem[];
  constexpr int CM = WM * CT * 16;
  constexpr int KC = GPC * kGroup;
  constexpr int pitch = KC / 8 + 1;
  const int G = K >> 7;
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % WN, wm = wave / WN;
  const int i = lane & 15, a = lane >> 4;
  const int m0 = blockIdx.y * CM;
  const int mrows = min(CM, M - m0);
  u32x4_t* xs = smem;
  float* cs = reinterpret_cast<float*>(smem + mrows * pitch);

  int rt[RB];
  bool rt_ok[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = (blockIdx.x * WN + wn) * RB + rb;
    rt_ok[rb] = r < ntiles;
    rt[rb] = min(r, ntiles - 1);
  }
  int colv[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) colv[ct] = min(wm * CT * 16 + ct * 16 + i, mrows - 1);

  f32x4_t acc[RB][CT];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rb][ct] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int g0 = 0; g0 < G; g0 += GPC) {
    const int ng = min(GPC, G - g0);
    // issue this chunk's weight and scale loads first; they fly during staging
    u32x4_t w[GPC][RB];
    float s[GPC][RB][4];
#pragma unroll
    for (int gl = 0; gl < GPC; ++gl) {
      if (gl < ng) {
        const int g = g0 + gl;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          if constexpr (PACKED) {
            const uint8_t* blk = W + (static_cast<size_t>(rt[rb]) * G + g) * kPackedBlock;
            w[gl][rb] = *reinterpret_cast<const u32x4_t*>(blk + lane * 16);
            scales_from_u32x2(*reinterpret_cast<const u32x2_t*>(blk + kPackedScaleOff + a * 8),
                              s[gl][rb]);
          } else {
            const int row = min(rt[rb] * kTileRows + i, N - 1);
            w[gl][rb] = *reinterpret_cast<const u32x4_t*>(
                W + static_cast<size_t>(row) * (K >> 1) + g * 64 + a * 16);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int srow = min(rt[rb] * kTileRows + 4 * a + r, N - 1);
              s[gl][rb][r] = half_bits_to_f32(S[static_cast<size_t>(srow) * G + g]);
            }
          }
        }
      }
    }
    __syncthreads();  // previous chunk's LDS reads are done
    stage_activations(xs, pitch, X, K, m0, mrows, g0 * kGroup, ng * kGroup);
    __syncthreads();
    stage_offsets(cs, GPC, xs, pitch, mrows, ng);
    __syncthreads();

#pragma unroll
    for (int gl = 0; gl < GPC; ++gl) {
      if (gl < ng) {
        f32x4_t tp[RB][CT];
        const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          u32x4_t A[RB];
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) A[rb] = decode_nibbles(w[gl][rb][d]);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            const u32x4_t B = xs[colv[ct] * pitch + gl * 16 + 4 * a + d];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              tp[rb][ct] = mfma16(A[rb], B, d == 0 ? zero : tp[rb][ct]);
          }
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const float c = cs[colv[ct] * GPC + gl];
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) group_epilogue(acc[rb][ct], tp[rb][ct], c, s[gl][rb]);
        }
      }
    }
  }

#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    if (!rt_ok[rb]) continue;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int cl = wm * CT * 16 + ct * 16 + i;
      if (cl < mrows)
        store_tile_column(Y, acc[rb][ct], static_cast<size_t>(m0 + cl) * N,
                          rt[rb] * kTileRows + 4 * a, N);
    }
  }
}

// ---------------------------------------------------------------------------
// Byte-wise fallback for misaligned bases (reference: int4gemv_scalar_bf16_
// kernel, src/kernels/int4_gemv_bf16.cu:174-213): one wave per (row, m),
// byte loads only, terms (q*s)*x in k order per lane, wave reduction.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t load_u16_bytes(const uint8_t* p) {
  return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
}

__global__ __launch_bounds__(256) void w4a16_bytewise_kernel(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ Sb,
    const uint8_t* __restrict__ Xb, uint8_t* __restrict__ Yb, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int m = blockIdx.y;
  if (row >= N) return;
  const int G = K >> 7;
  const uint8_t* wrow = W + static_cast<size_t>(row) * (K >> 1);
  const uint8_t* srow = Sb + static_cast<size_t>(row) * G * 2;
  const uint8_t* xrow = Xb + static_cast<size_t>(m) * K * 2;
  float acc = 0.0f;
  for (int b = lane; b < (K >> 1); b += 64) {
    const uint32_t byte = wrow[b];
    const float s = half_bits_to_f32(load_u16_bytes(srow + 2 * (b >> 6)));
    const int lo = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>(byte << 4))) >> 4;
    const int hi = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>(byte))) >> 4;
    const float x0 = bf16_lo(load_u16_bytes(xrow + 4 * b));
    const float x1 = bf16_lo(load_u16_bytes(xrow + 4 * b + 2));
    acc += (static_cast<float>(lo) * s) * x0;
    acc += (static_cast<float>(hi) * s) * x1;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) {
    const uint32_t y = f32_to_bf16_rne(acc);
    uint8_t* yp = Yb + (static_cast<size_t>(m) * N + row) * 2;
    yp[0] = static_cast<uint8_t>(y & 0xFF);
    yp[1] = static_cast<uint8_t>(y >> 8);
  }
}

// ---------------------------------------------------------------------------
// Dequantization through decode_nibbles (bit-exact check of the decoder).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void w4a16_dequant_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    int8_t* __restrict__ qo, float* __restrict__ wo, int N, int K) {
  const size_t dwords_per_row = static_cast<size_t>(K) >> 3;
  const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= dwords_per_row * N) return;
  const size_t n = idx / dwords_per_row;
  const size_t dw = idx - n * dwords_per_row;
  const uint32_t w = reinterpret_cast<const uint32_t*>(W + n * (K >> 1))[dw];
  const u32x4_t pairs = decode_nibbles(w);
  const float s = half_bits_to_f32(S[n * (K >> 7) + (dw >> 4)]);
  const size_t k0 = n * K + dw * 8;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float e0 = (bf16_lo(pairs[p]) - 1.5f) * 16.0f;  // element k0 + p
    const float e1 = (bf16_hi(pairs[p]) - 1.5f) * 16.0f;  // element k0 + p + 4
    if (qo) {
      qo[k0 + p] = static_cast<int8_t>(e0);
      qo[k0 + p + 4] = static_cast<int8_t>(e1);
    }
    if (wo) {
      wo[k0 + p] = e0 * s;
      wo[k0 + p + 4] = e1 * s;
    }
  }
}

// ---------------------------------------------------------------------------
// Load-time repack: file layout -> tile-major blocks of 1056 bytes per
// (16-row tile, group): bytes [16l, 16l+16) hold row l%16, k-bytes
// [16(l/16), +16) of the group (what MFMA lane l loads); bytes [1024, 1056)
// hold the group's 16 row scales (fp16) in row order. Rows >= N are zero.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void w4a16_repack_kernel(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ Sb,
    uint8_t* __restrict__ P, int N, int K) {
  const int G = K >> 7;
  const size_t units_per_block = kPackedBlock / 16;  // 66
  const size_t nunits = static_cast<size_t>((N + 15) / 16) * G * units_per_block;
  const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= nunits) return;
  const size_t blk = idx / units_per_block;
  const int j = static_cast<int>(idx - blk * units_per_block);
  const int rt = static_cast<int>(blk / G);
  const int g = static_cast<int>(blk - static_cast<size_t>(rt) * G);
  uint8_t out[16];
  if (j < 64) {
    const int n = rt * 16 + (j & 15);
    const int a = j >> 4;
    for (int b = 0; b < 16; ++b)
      out[b] = (n < N) ? W[static_cast<size_t>(n) * (K >> 1) + g * 64 + a * 16 + b] : 0;
  } else {
    const int r0 = (j - 64) * 8;
    for (int r = 0; r < 8; ++r) {
      const int n = rt * 16 + r0 + r;
      const size_t so = (static_cast<size_t>(n) * G + g) * 2;
      out[2 * r] = (n < N) ? Sb[so] : 0;
      out[2 * r + 1] = (n < N) ? Sb[so + 1] : 0;
    }
  }
  u32x4_t v;
  for (int q = 0; q < 4; ++q)
    v[q] = static_cast<uint32_t>(out[4 * q]) | (static_cast<uint32_t>(out[4 * q + 1]) << 8) |
           (static_cast<uint32_t>(out[4 * q + 2]) << 16) |
           (static_cast<uint32_t>(out[4 * q + 3]) << 24);
  reinterpret_cast<u32x4_t*>(P)[idx] = v;
}

// ---------------------------------------------------------------------------
// host launch layer
// ---------------------------------------------------------------------------

constexpr size_t kLdsBudget = 64 * 1024;

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_shape(int N, int K, int M) {
  if (N < 1 || M < 1 || K <= 0 || K % kGroup != 0) return CUDALM_W4A16_EINVAL;
  // 32-bit tile/group indices inside the kernels
  if (static_cast<long long>(N) + 16 > (1LL << 30) || K > (1 << 24) ||
      static_cast<long long>(M) > 65535LL * 128)
    return CUDALM_W4A16_ERANGE;
  return CUDALM_W4A16_OK;
}

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? CUDALM_W4A16_OK : CUDALM_W4A16_ELAUNCH;
}

size_t stream_lds_bytes(int K, int M) {
  const int G = K / kGroup;
  const size_t x = static_cast<size_t>(M) * (K / 8 + 1) * 16;
  const size_t c = static_cast<size_t>((M * G + 3) & ~3) * 4;
  const size_t s = static_cast<size_t>(kStreamWaves) * kStreamUnit * kTileRows * 2;
  return x + c + s;
}

template <bool PACKED>
int launch_stream(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                  int K, int M, hipStream_t stream) {
  const size_t lds = stream_lds_bytes(K, M);
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int want = (ntiles + kStreamWaves - 1) / kStreamWaves;
  const int cap = cu_count() * 4;
  const int grid = want < cap ? want : cap;
  hipLaunchKernelGGL(w4a16_stream_kernel<PACKED>, dim3(grid), dim3(kStreamWaves * 64), lds,
                     stream, W, S, X, Y, N, K, M);
  return launch_status();
}

template <int RB, int CT, int WN, int WM, int GPC, bool PACKED>
int launch_tile(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                int K, int M, hipStream_t stream) {
  constexpr int CM = WM * CT * 16;
  constexpr int KC = GPC * kGroup;
  const int mrows = M < CM ? M : CM;
  const size_t lds = static_cast<size_t>(mrows) * (KC / 8 + 1) * 16 + static_cast<size_t>(mrows) * GPC * 4;
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int gx = (ntiles + WN * RB - 1) / (WN * RB);
  const int gy = (M + CM - 1) / CM;
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  hipLaunchKernelGGL((w4a16_tile_kernel<RB, CT, WN, WM, GPC, PACKED>), dim3(gx, gy),
                     dim3(WN * WM * 64), lds, stream, W, S, X, Y, N, K, M);
  return launch_status();
}

int launch_bytewise(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                    int K, int M, hipStream_t stream) {
  if (M > 65535) return CUDALM_W4A16_ERANGE;
  hipLaunchKernelGGL(w4a16_bytewise_kernel, dim3((N + 3) / 4, M), dim3(256), 0, stream, W,
                     reinterpret_cast<const uint8_t*>(S), reinterpret_cast<const uint8_t*>(X),
                     reinterpret_cast<uint8_t*>(Y), N, K);
  return launch_status();
}

template <bool PACKED>
int dispatch(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N, int K,
             int M, int variant, hipStream_t stream) {
  if (variant == CUDALM_W4A16_VARIANT_AUTO) {
    if (M <= 16 && stream_lds_bytes(K, M) <= kLdsBudget)
      variant = CUDALM_W4A16_VARIANT_STREAM;
    else if (M <= 16)
      variant = CUDALM_W4A16_VARIANT_TILE16;
    else if (M <= 32)
      variant = CUDALM_W4A16_VARIANT_TILE32;
    else
      variant = CUDALM_W4A16_VARIANT_PREFILL;
  }
  switch (variant) {
    case CUDALM_W4A16_VARIANT_STREAM:
      if (M > 16 || stream_lds_bytes(K, M) > kLdsBudget) return CUDALM_W4A16_EINVAL;
      return launch_stream<PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_TILE16:
      return launch_tile<1, 1, 4, 1, 8, PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_TILE32:
      return launch_tile<1, 2, 4, 1, 8, PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_PREFILL:
      return launch_tile<4, 4, 2, 2, 2, PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_BYTEWISE:
      if (PACKED) return CUDALM_W4A16_EVARIANT;
      return launch_bytewise(W, S, X, Y, N, K, M, stream);
    default:
      return CUDALM_W4A16_EVARIANT;
  }
}

template <typename F>
int regs_of(F kernel) {
  hipFuncAttributes attr;
  if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kernel)) != hipSuccess) return -1;
  return attr.numRegs;
}

}  // namespace

extern "C" {

int cudalm_w4a16_version(void) { return 100; }

const char* cudalm_w4a16_strerror(int code) {
  switch (code) {
    case CUDALM_W4A16_OK: return "ok";
    case CUDALM_W4A16_EINVAL: return "invalid shape: requires N >= 1, M >= 1, K > 0, K % 128 == 0";
    case CUDALM_W4A16_ENULL: return "null pointer argument";
    case CUDALM_W4A16_EALIGN: return "prepacked weight or activation base not 16-byte aligned";
    case CUDALM_W4A16_ELAUNCH: return "HIP kernel launch failed";
    case CUDALM_W4A16_ERANGE: return "shape exceeds the kernels' index range";
    case CUDALM_W4A16_EVARIANT: return "unknown or inapplicable kernel variant";
    default: return "unknown error code";
  }
}

int cudalm_w4a16_gemv_bf16_variant(const uint8_t* weight, const uint16_t* scale,
                                   const uint16_t* x, uint16_t* y, int N, int K, int M,
                                   int variant, hipStream_t stream) {
  if (int rc = check_shape(N, K, M)) return rc;
  if (!weight || !scale || !x || !y) return CUDALM_W4A16_ENULL;
  // The vectorized kernels need 16 B aligned weight rows and activation rows
  // (K % 128 == 0 keeps every row aligned once the base is) and 2 B aligned
  // scales / outputs; anything else takes the byte-wise kernel.
  const bool vec_ok = aligned(weight, 16) && aligned(x, 16) && aligned(scale, 2) && aligned(y, 2);
  if (!vec_ok) {
    if (variant != CUDALM_W4A16_VARIANT_AUTO && variant != CUDALM_W4A16_VARIANT_BYTEWISE)
      return CUDALM_W4A16_EVARIANT;
    variant = CUDALM_W4A16_VARIANT_BYTEWISE;
  }
  return dispatch<false>(weight, scale, x, y, N, K, M, variant, stream);
}

int cudalm_w4a16_gemv_bf16(const uint8_t* weight, const uint16_t* scale, const uint16_t* x,
                           uint16_t* y, int N, int K, int M, hipStream_t stream) {
  return cudalm_w4a16_gemv_bf16_variant(weight, scale, x, y, N, K, M, CUDALM_W4A16_VARIANT_AUTO,
                                        stream);
}

size_t cudalm_w4a16_packed_bytes(int N, int K) {
  if (N < 1 || K <= 0 || K % kGroup != 0) return 0;
  return static_cast<size_t>((N + 15) / 16) * (K / kGroup) * kPackedBlock;
}

int cudalm_w4a16_repack(const uint8_t* weight, const uint16_t* scale, void* packed, int N, int K,
                        hipStream_t stream) {
  if (int rc = check_shape(N, K, 1)) return rc;
  if (!weight || !scale || !packed) return CUDALM_W4A16_ENULL;
  if (!aligned(packed, 16)) return CUDALM_W4A16_EALIGN;
  const size_t units = cudalm_w4a16_packed_bytes(N, K) / 16;
  const size_t blocks = (units + 255) / 256;
  if (blocks > 0x7FFFFFFFu) return CUDALM_W4A16_ERANGE;
  hipLaunchKernelGGL(w4a16_repack_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     weight, reinterpret_cast<const uint8_t*>(scale),
                     reinterpret_cast<uint8_t*>(packed), N, K);
  return launch_status();
}

int cudalm_w4a16_gemv_bf16_prepacked_variant(const void* packed, const uint16_t* x, uint16_t* y,
                                             int N, int K, int M, int variant,
                                             hipStream_t stream) {
  if (int rc = check_shape(N, K, M)) return rc;
  if (!packed || !x || !y) return CUDALM_W4A16_ENULL;
  if (!aligned(packed, 16) || !aligned(x, 16) || !aligned(y, 2)) return CUDALM_W4A16_EALIGN;
  return dispatch<true>(reinterpret_cast<const uint8_t*>(packed), nullptr, x, y, N, K, M, variant,
                        stream);
}

int cudalm_w4a16_gemv_bf16_prepacked(const void* packed, const uint16_t* x, uint16_t* y, int N,
                                     int K, int M, hipStream_t stream) {
  return cudalm_w4a16_gemv_bf16_prepacked_variant(packed, x, y, N, K, M,
                                                  CUDALM_W4A16_VARIANT_AUTO, stream);
}

int cudalm_w4a16_dequant_f32(const uint8_t* weight, const uint16_t* scale, int8_t* q_out,
                             float* w_out, int N, int K, hipStream_t stream) {
  if (int rc = check_shape(N, K, 1)) return rc;
  if (!weight || !scale) return CUDALM_W4A16_ENULL;
  if (!aligned(weight, 4) || !aligned(scale, 2) || (w_out && !aligned(w_out, 4)))
    return CUDALM_W4A16_EALIGN;
  const size_t threads = static_cast<size_t>(N) * (K / 8);
  const size_t blocks = (threads + 255) / 256;
  if (blocks > 0x7FFFFFFFu) return CUDALM_W4A16_ERANGE;
  hipLaunchKernelGGL(w4a16_dequant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, weight, scale, q_out, w_out, N, K);
  return launch_status();
}

int cudalm_w4a16_kernel_regs(int variant) {
  switch (variant) {
    case CUDALM_W4A16_VARIANT_AUTO:
    case CUDALM_W4A16_VARIANT_STREAM: return regs_of(w4a16_stream_kernel<true>);
    case CUDALM_W4A16_VARIANT_TILE16: return regs_of(w4a16_tile_kernel<1, 1, 4, 1, 8, true>);
    case CUDALM_W4A16_VARIANT_TILE32: return regs_of(w4a16_tile_kernel<1, 2, 4, 1, 8, true>);
    case CUDALM_W4A16_VARIANT_PREFILL: return regs_of(w4a16_tile_kernel<4, 4, 2, 2, 2, true>);
    case CUDALM_W4A16_VARIANT_BYTEWISE: return regs_of(w4a16_bytewise_kernel);
    default: return -1;
  }
}

}  // extern "C"
