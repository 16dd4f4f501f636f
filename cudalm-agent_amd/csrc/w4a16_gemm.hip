// Prefill-chunk W4A16 GEMM on 32 x 32 MFMA tiles (MI355X, gfx950).
//
// Contract (reference: tests/cuda/test_int4_gemv_bf16.cpp:54-69 applied row
// by row; the reference itself runs prefill one token at a time,
// src/runtime/qwen35_generator.cpp:107-125):
//   y[m,n] = bf16_rne( sum_k q[n,k] * f32(s[n,k/128]) * f32(x[m,k]) ).
//
// Matrix-core mapping. v_mfma_f32_32x32x16_bf16 multiplies 32 activation
// rows (A, m) by 32 weight rows (B, n) over 16 k: lane l = 32h + j holds
// A row j / B column j at k-block h (8 k) of the instruction, and D rows
// 8(r/4) + 4h + r%4 of column j in its 16 accumulators. One decoded weight
// dword (8 nibbles -> 4 bf16 pairs) therefore feeds 32 activation rows per
// instruction, twice as many as the 16 x 16 x 32 tiles of the decode
// kernels, and a wave that owns MT 32-row activation tiles feeds it to MT
// instructions: the decode VALU per FLOP is 1/(2 MT) of the 16 x 16 path.
//
// Same bits as every other kernel of the library. A 16 x 16 x 32 step over
// the k-blocks (b0, b1, b2, b3) of its four lane rows gives exactly the fp32
// result of two 32 x 32 x 16 steps, the first over (b0, b1) and the second
// over (b2, b3) (measured on gfx950: 0 of 1,048,576 outputs differ, random
// bf16 A, 1.5 + q/16 weights, zero and nonzero accumulators). So group g's
// chain runs, for each 16 x 16 step d = 0..3 of the decode kernels (lane
// row a holds k = 32a + 8d .. +7), the two halves e = 0, 1 over k-blocks
// 32(2e) + 8d and 32(2e+1) + 8d; it is seeded with the same offset chain
// (-1.5 * sum x per row and group, computed with the decode kernels' four
// 16 x 16 x 32 MFMAs into an LDS table); the epilogue is the canonical
// part = fma(s[n, g], tmp, part) in group order from 0 within an 8-group
// unit, total = 0 + part_u in unit order, y = bf16_rne(16 * total).
//
// Work decomposition. A workgroup of WVN waves owns TN = 32 WVN weight rows
// and TM = 32 MT activation rows. Per 8-group unit (1024 k): the tile's x
// is staged once into LDS in pair order, the waves split the offset chains
// of the unit's (group, 16-row) pairs into an LDS table, and each wave
// decodes its 32 rows' weights once per k-block and runs MT chains per
// group. Weights of the unit are loaded before the x staging completes.
// At K = 1024 (one unit) w4a16_gemm32_split_kernel runs instead: the
// unit's groups are split over two wave sets, which hand the canonical fma
// chain from one to the other through LDS.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "cudalm_w4a16.h"
#include "hip_common.h"
#include "w4a16_device.h"

namespace cudalm_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// D = A (32 rows x 16 k) * B (16 k x 32 cols) + C, bf16 in, fp32 accumulate.
__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

constexpr int kPB = kUnit * 16 + 1;  // LDS row pitch of one unit of x, 16-byte blocks (padded)

template <int WVN, int MT>
constexpr size_t gemm32_lds_bytes() {
  return static_cast<size_t>(32 * MT) * kPB * 16 + static_cast<size_t>(kUnit) * 32 * MT * 4;
}

// WVN waves along n, each owning NB 32-row weight tiles; MT 32-row
// activation tiles per workgroup (every wave runs all of them).
template <int WVN, int MT, int NB, bool PACKED, bool SVEC>
__global__ __launch_bounds__(WVN * 64) void w4a16_gemm32_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int K, int M) {
  constexpr int NT = WVN * 64;
  constexpr int TM = 32 * MT;
  extern __shared__ u32x4_t lds[];  // x [TM][kPB], then the offset table [8 groups][TM] f32
  u32x4_t* xs = lds;
  float* corr = reinterpret_cast<float*>(lds + TM * kPB);

  const int G = K >> 7;
  const int U = (G + kUnit - 1) / kUnit;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int tid = static_cast<int>(threadIdx.x);
  const int j = lane & 31, h = lane >> 5;      // 32 x 32 operand lane: row / column j, k-block h
  const int i16 = lane & 15, a16 = lane >> 4;  // 16 x 16 operand lane (offset chains)
  const int m0 = blockIdx.y * TM;
  const int mrows = min(TM, M - m0);
  const int nbase = (blockIdx.x * WVN + wave) * 32 * NB;  // this wave's first weight row
  const bool wave_ok = nbase < N;

  // lane addresses at group 0 of weight row n = nbase + 32 nb + j: chunk
  // a = h (k 32h .. 32h+31 of a group) and chunk a = 2 + h
  const uint8_t* w_lo[NB];
  const uint8_t* w_hi[NB];
  const uint8_t* s_row[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = nbase + 32 * nb + j;
    if constexpr (PACKED) {
      const int t16 = min(n, N - 1) >> 4, r16 = n & 15;
      const uint8_t* tile = W + static_cast<size_t>(t16) * packed_tile_bytes(G);
      w_lo[nb] = tile + 16 * (16 * h + r16);
      w_hi[nb] = tile + 16 * (16 * (2 + h) + r16);
      s_row[nb] = tile + static_cast<size_t>(G) * 1024 + r16 * packed_scale_pitch(G);
    } else {
      const int row = min(n, N - 1);
      w_lo[nb] = W + static_cast<size_t>(row) * (K >> 1) + 16 * h;
      w_hi[nb] = w_lo[nb] + 32;
      s_row[nb] = reinterpret_cast<const uint8_t*>(S + static_cast<size_t>(row) * G);
    }
  }
  constexpr int kStep = PACKED ? 1024 : 64;  // bytes between groups of one lane

  const f32x16_t zero16 = {};
  f32x16_t acc[NB][MT];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nb][mt] = zero16;

  constexpr int NBLK = TM * kUnit * 16;  // 16-byte x blocks of one unit
  static_assert(NBLK % NT == 0, "staging covers the tile exactly");
  constexpr int BPT = NBLK / NT;         // x blocks staged per thread per unit
  constexpr int RS = NT / (kUnit * 16);  // rows staged per pass (a thread keeps one block column)
  static_assert(NT % (kUnit * 16) == 0, "a thread keeps one block column");
  constexpr int NCH = kUnit * 2 * MT;    // offset chains per unit (group, 16-row tile)
  constexpr int CPW = (NCH + WVN - 1) / WVN;  // offset chains per wave

  for (int u = 0; u < U; ++u) {
    const int g0 = u * kUnit;
    const int gn = min(kUnit, G - g0);
    // the unit's activations first (staged, then the offset table), then
    // this wave's weights and scales; loads return in issue order
    const int b = tid & (kUnit * 16 - 1);
    const int r0 = tid / (kUnit * 16);
    u32x4_t v[BPT];
    {
      const uint16_t* xcol = X + static_cast<size_t>(m0) * K + min(g0 * kGroup + 8 * b, K - 8);
#pragma unroll
      for (int q = 0; q < BPT; ++q)
        v[q] = *reinterpret_cast<const u32x4_t*>(
            xcol + static_cast<size_t>(min(r0 + q * RS, mrows - 1)) * K);
    }
    u32x4_t wl[NB][kUnit], wh[NB][kUnit];
    uint32_t sc[NB][kUnit / 2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int gg = 0; gg < kUnit; ++gg) {
        const size_t off = static_cast<size_t>(min(g0 + gg, G - 1)) * kStep;
        wl[nb][gg] = *reinterpret_cast<const u32x4_t*>(w_lo[nb] + off);
        wh[nb][gg] = *reinterpret_cast<const u32x4_t*>(w_hi[nb] + off);
      }
      if constexpr (PACKED || SVEC) {
        const u32x4_t sv = *reinterpret_cast<const u32x4_t*>(s_row[nb] + 2 * g0);
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[nb][q] = sv[q];
      } else {
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(s_row[nb]);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sc[nb][q] = static_cast<uint32_t>(srow[min(g0 + 2 * q, G - 1)]) |
                      (static_cast<uint32_t>(srow[min(g0 + 2 * q + 1, G - 1)]) << 16);
      }
    }
    if (u > 0) __syncthreads();  // the previous unit's readers are done
    {
      u32x4_t* xdst = xs + r0 * kPB + b;
#pragma unroll
      for (int q = 0; q < BPT; ++q) xdst[q * RS * kPB] = pair_order(v[q]);
    }
    __syncthreads();
    // offset table: chains (group, 16-row activation tile) split over the
    // waves, the decode kernels' four 16 x 16 x 32 MFMAs each; a wave's
    // chains are independent and run side by side
    {
      u32x4_t xo[CPW][4];
#pragma unroll
      for (int q = 0; q < CPW; ++q) {
        const int c = min(wave + q * WVN, NCH - 1);
        const int gg = c / (2 * MT), st = c - gg * (2 * MT);
        const u32x4_t* xg = xs + (st * 16 + i16) * kPB + gg * 16 + 4 * a16;
#pragma unroll
        for (int d = 0; d < 4; ++d) xo[q][d] = xg[d];
      }
#pragma unroll
      for (int q = 0; q < CPW; ++q) {
        const int c = wave + q * WVN;
        const f32x4_t o = group_offset(xo[q]);
        if (c < NCH && i16 == 0) {
          const int gg = c / (2 * MT), st = c - gg * (2 * MT);
          *reinterpret_cast<f32x4_t*>(corr + gg * TM + st * 16 + 4 * a16) = o;
        }
      }
    }
    __syncthreads();
    if (!wave_ok) continue;

    f32x16_t part[NB][MT];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) part[nb][mt] = zero16;
    // one group: offset-seeded chains, then the scale fma into part
    auto group = [&](int gg) {
      u32x4_t xa[4][2][MT];
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            xa[d][e][mt] = xs[(mt * 32 + j) * kPB + gg * 16 + 4 * (2 * e + h) + d];
      f32x16_t t[NB][MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // seed: D row 8(r/4) + 4h + r%4 of column j holds that row's offset
        const float* cr = corr + gg * TM + mt * 32 + 4 * h;
        f32x16_t o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4_t o4 = *reinterpret_cast<const f32x4_t*>(cr + 8 * q);
#pragma unroll
          for (int r = 0; r < 4; ++r) o[4 * q + r] = o4[r];
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) t[nb][mt] = o;
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const u32x4_t B = decode_nibbles<PACKED>(e == 0 ? wl[nb][gg][d] : wh[nb][gg][d]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) t[nb][mt] = mfma32(xa[d][e][mt], B, t[nb][mt]);
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const float s = half_bits_to_f32((sc[nb][gg >> 1] >> (16 * (gg & 1))) & 0xFFFFu);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            part[nb][mt][r] = __builtin_fmaf(s, t[nb][mt][r], part[nb][mt][r]);
      }
    };
    if (gn == kUnit) {
#pragma unroll
      for (int gg = 0; gg < kUnit; ++gg) group(gg);
    } else {
#pragma unroll
      for (int gg = 0; gg < kUnit; ++gg)
        if (gg < gn) group(gg);
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nb][mt] = acc[nb][mt] + part[nb][mt];
  }
  if (!wave_ok) return;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = nbase + 32 * nb + j;
    if (n >= N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < mrows) {
          // a NaN sum (infinite or NaN activations, overflow) is recomputed
          // by the reference loop, which keeps the reference's semantics
          float v = 16.0f * acc[nb][mt][r];
          if (__builtin_expect(v != v, 0))
            v = w4a16_ref_dot<PACKED>(W, S, K, n, X + static_cast<size_t>(m0 + m) * K);
          Y[static_cast<size_t>(m0 + m) * N + n] = static_cast<uint16_t>(f32_to_bf16_rne(v));
        }
      }
  }
}

// K = 1024 (one 8-group unit): the unit's groups split over two wave sets.
// A workgroup of 2 x WVN waves owns 32 WVN weight rows and 32 activation
// rows; wave (ks, wn) loads and decodes the weights of groups 4 ks .. 4 ks + 3
// of rows 32 wn .. 32 wn + 31 and runs their offset-seeded chains. Set 0
// folds its four chain results into part = fma(s, tmp, part) in group order
// and hands part to set 1 through LDS; set 1 holds its four results in
// registers and continues the same fma chain with groups 4..7, then stores.
// The arithmetic is that of w4a16_gemm32_kernel, step for step; each wave
// has half the weight loads and half the chains on its critical path.
constexpr int kSplitHalf = kUnit / 2;  // groups per wave set

// File layout: each wave loads its rows' 256-byte run of the set's four
// groups in whole lines (load q: rows 4q .. 4q + 3, lane l: bytes 16 (l % 16)
// of row 4q + l / 16) and re-lays them out for the MFMA lanes through a
// per-wave LDS staging area, half the run at a time (rows of 144 bytes).
// With 2-wave sets the staging would leave room for one workgroup per CU
// instead of two, so those keep 32-byte loads straight into the lanes.
constexpr int kSplitStagePitch = 144;

template <int WVN, bool PACKED>
constexpr bool split_staged() {
  return !PACKED && WVN >= 4;
}

// 4-wave sets without staging hand part over through the activation buffer
// (after a barrier every reader of it has passed): 67 KB of LDS, two
// workgroups per CU.
template <int WVN, bool PACKED>
constexpr bool split_alias() {
  return WVN == 4 && !split_staged<WVN, PACKED>();
}

template <int WVN, bool PACKED>
constexpr size_t gemm32_split_lds_bytes() {
  // the part hand-over (WVN x 4 KB) reuses the file layout's staging area
  return gemm32_lds_bytes<WVN, 1>() +
         (split_staged<WVN, PACKED>() ? static_cast<size_t>(2 * WVN) * 32 * kSplitStagePitch
          : split_alias<WVN, PACKED>() ? static_cast<size_t>(0)
                                       : static_cast<size_t>(WVN) * 64 * 16 * 4);
}

template <int WVN, bool PACKED, bool SVEC>
__global__ __launch_bounds__(WVN * 2 * 64) void w4a16_gemm32_split_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int M) {
  constexpr int K = kUnit * kGroup;
  constexpr int G = kUnit;
  constexpr int NW = 2 * WVN;  // waves per workgroup
  constexpr int NT = NW * 64;
  constexpr int TM = 32;
  constexpr bool STAGED = split_staged<WVN, PACKED>();
  extern __shared__ u32x4_t lds[];  // x [TM][kPB], offset table [8][TM] f32, part exchange
  u32x4_t* xs = lds;
  float* corr = reinterpret_cast<float*>(lds + TM * kPB);
  uint8_t* stage = reinterpret_cast<uint8_t*>(corr + kUnit * TM);
  constexpr bool ALIAS = split_alias<WVN, PACKED>();
  f32x4_t* xchg = reinterpret_cast<f32x4_t*>(ALIAS ? reinterpret_cast<uint8_t*>(lds) : stage);

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int ks = wave / WVN, wn = wave - ks * WVN;
  const int tid = static_cast<int>(threadIdx.x);
  const int j = lane & 31, h = lane >> 5;
  const int i16 = lane & 15, a16 = lane >> 4;
  const int m0 = blockIdx.y * TM;
  const int mrows = min(TM, M - m0);
  const int n = (blockIdx.x * WVN + wn) * 32 + j;
  const bool wave_ok = (blockIdx.x * WVN + wn) * 32 < N;
  const int gb = ks * kSplitHalf;  // this wave set's first group

  // activations first (loads return in issue order), then the weights and
  // scales of this wave set's groups
  constexpr int NBLK = TM * kUnit * 16;
  static_assert(NBLK % NT == 0 && NT % (kUnit * 16) == 0, "staging covers the tile exactly");
  constexpr int BPT = NBLK / NT;
  constexpr int RS = NT / (kUnit * 16);
  const int b = tid & (kUnit * 16 - 1);
  const int r0 = tid / (kUnit * 16);
  u32x4_t v[BPT];
  {
    const uint16_t* xcol = X + static_cast<size_t>(m0) * K + 8 * b;
#pragma unroll
    for (int q = 0; q < BPT; ++q)
      v[q] = *reinterpret_cast<const u32x4_t*>(xcol +
                                               static_cast<size_t>(min(r0 + q * RS, mrows - 1)) * K);
  }
  u32x4_t wl[kSplitHalf], wh[kSplitHalf];
  u32x4_t raw[8];  // file layout: the whole-line loads, before the re-layout
  uint32_t sc[kSplitHalf / 2];
  {
    const int row = min(n, N - 1);
    const uint8_t* s_row;
    if constexpr (PACKED) {
      const uint8_t* tile = W + static_cast<size_t>(row >> 4) * packed_tile_bytes(G);
      const uint8_t* w_lo = tile + 16 * (16 * h + (row & 15));
      s_row = tile + static_cast<size_t>(G) * 1024 + (row & 15) * packed_scale_pitch(G);
#pragma unroll
      for (int gg = 0; gg < kSplitHalf; ++gg) {
        wl[gg] = *reinterpret_cast<const u32x4_t*>(w_lo + (gb + gg) * 1024);
        wh[gg] = *reinterpret_cast<const u32x4_t*>(w_lo + 16 * 32 + (gb + gg) * 1024);
      }
    } else if constexpr (!STAGED) {
      const uint8_t* w_lo = W + static_cast<size_t>(row) * (K >> 1) + 16 * h;
      s_row = reinterpret_cast<const uint8_t*>(S + static_cast<size_t>(row) * G);
#pragma unroll
      for (int gg = 0; gg < kSplitHalf; ++gg) {
        wl[gg] = *reinterpret_cast<const u32x4_t*>(w_lo + (gb + gg) * 64);
        wh[gg] = *reinterpret_cast<const u32x4_t*>(w_lo + 32 + (gb + gg) * 64);
      }
    } else {
      s_row = reinterpret_cast<const uint8_t*>(S + static_cast<size_t>(row) * G);
      const int rbase = (blockIdx.x * WVN + wn) * 32 + (lane >> 4);
      const uint8_t* wcol = W + gb * 64 + 16 * (lane & 15);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        raw[q] = *reinterpret_cast<const u32x4_t*>(
            wcol + static_cast<size_t>(min(rbase + 4 * q, N - 1)) * (K >> 1));
    }
    if constexpr (PACKED || SVEC) {
      const uint2 sv = *reinterpret_cast<const uint2*>(s_row + 2 * gb);
      sc[0] = sv.x;
      sc[1] = sv.y;
    } else {
      const uint16_t* srow = reinterpret_cast<const uint16_t*>(s_row);
#pragma unroll
      for (int q = 0; q < kSplitHalf / 2; ++q)
        sc[q] = static_cast<uint32_t>(srow[gb + 2 * q]) |
                (static_cast<uint32_t>(srow[gb + 2 * q + 1]) << 16);
    }
  }
  {
    u32x4_t* xdst = xs + r0 * kPB + b;
#pragma unroll
    for (int q = 0; q < BPT; ++q) xdst[q * RS * kPB] = pair_order(v[q]);
  }
  __syncthreads();
  // offset table: 16 chains (group, 16-row tile) split over the waves
  {
    constexpr int NCH = kUnit * 2;
    constexpr int CPW = (NCH + NW - 1) / NW;
    u32x4_t xo[CPW][4];
#pragma unroll
    for (int q = 0; q < CPW; ++q) {
      const int c = min(wave + q * NW, NCH - 1);
      const u32x4_t* xg = xs + ((c & 1) * 16 + i16) * kPB + (c >> 1) * 16 + 4 * a16;
#pragma unroll
      for (int d = 0; d < 4; ++d) xo[q][d] = xg[d];
    }
#pragma unroll
    for (int q = 0; q < CPW; ++q) {
      const int c = wave + q * NW;
      const f32x4_t o = group_offset(xo[q]);
      if (c < NCH && i16 == 0)
        *reinterpret_cast<f32x4_t*>(corr + (c >> 1) * TM + (c & 1) * 16 + 4 * a16) = o;
    }
  }
  __syncthreads();

  if constexpr (STAGED) {
    // re-lay the wave's rows out for the MFMA lanes: lane (j, h) takes
    // 16-byte chunks 4 gq + h (groups' k 32h .. 32h + 31) and 4 gq + 2 + h
    // of row j
    uint8_t* st = stage + wave * 32 * kSplitStagePitch;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      if (((lane >> 3) & 1) == hh) {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          *reinterpret_cast<u32x4_t*>(st + (4 * q + (lane >> 4)) * kSplitStagePitch +
                                      (lane & 7) * 16) = raw[q];
      }
      wave_lds_sync();
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        wl[2 * hh + g2] =
            *reinterpret_cast<const u32x4_t*>(st + j * kSplitStagePitch + (4 * g2 + h) * 16);
        wh[2 * hh + g2] =
            *reinterpret_cast<const u32x4_t*>(st + j * kSplitStagePitch + (4 * g2 + 2 + h) * 16);
      }
      wave_lds_sync();
    }
  }

  // chain results of this wave set's groups
  f32x16_t t[kSplitHalf];
  if (wave_ok) {
#pragma unroll
    for (int gq = 0; gq < kSplitHalf; ++gq) {
      const int gg = gb + gq;
      u32x4_t xa[4][2];
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int e = 0; e < 2; ++e) xa[d][e] = xs[j * kPB + gg * 16 + 4 * (2 * e + h) + d];
      const float* cr = corr + gg * TM + 4 * h;
      f32x16_t acc;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t o4 = *reinterpret_cast<const f32x4_t*>(cr + 8 * q);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[4 * q + r] = o4[r];
      }
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int e = 0; e < 2; ++e)
          acc = mfma32(xa[d][e], decode_nibbles<PACKED>(e == 0 ? wl[gq][d] : wh[gq][d]), acc);
      t[gq] = acc;
    }
  }
  const auto scale = [&](int gq) {
    return half_bits_to_f32((sc[gq >> 1] >> (16 * (gq & 1))) & 0xFFFFu);
  };
  f32x4_t* slot = xchg + wn * 4 * 64 + lane;
  f32x16_t part = {};
  if (ks == 0 && wave_ok) {
#pragma unroll
    for (int gq = 0; gq < kSplitHalf; ++gq) {
      const float s = scale(gq);
#pragma unroll
      for (int r = 0; r < 16; ++r) part[r] = __builtin_fmaf(s, t[gq][r], part[r]);
    }
  }
  // every wave is done with its staging rows / the activations
  if constexpr (STAGED || ALIAS) __syncthreads();
  if (ks == 0 && wave_ok) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      slot[q * 64] = f32x4_t{part[4 * q], part[4 * q + 1], part[4 * q + 2], part[4 * q + 3]};
  }
  __syncthreads();
  if (ks == 0 || !wave_ok || n >= N) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4_t p4 = slot[q * 64];
#pragma unroll
    for (int r = 0; r < 4; ++r) part[4 * q + r] = p4[r];
  }
#pragma unroll
  for (int gq = 0; gq < kSplitHalf; ++gq) {
    const float s = scale(gq);
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = __builtin_fmaf(s, t[gq][r], part[r]);
  }
  // one unit: total = 0 + part
  const f32x16_t zero16 = {};
  const f32x16_t total = zero16 + part;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = 8 * (r >> 2) + 4 * h + (r & 3);
    if (m < mrows) {
      float val = 16.0f * total[r];
      if (__builtin_expect(val != val, 0))
        val = w4a16_ref_dot<PACKED>(W, S, K, n, X + static_cast<size_t>(m0 + m) * K);
      Y[static_cast<size_t>(m0 + m) * N + n] = static_cast<uint16_t>(f32_to_bf16_rne(val));
    }
  }
}

template <int WVN, bool PACKED>
int launch_gemm32_split(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                        int M, hipStream_t stream) {
  const size_t lds = gemm32_split_lds_bytes<WVN, PACKED>();
  const int gx = (N + 32 * WVN - 1) / (32 * WVN);
  const int gy = (M + 31) / 32;
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  const bool svec = !PACKED && aligned(S, 8);
  auto kern = svec ? w4a16_gemm32_split_kernel<WVN, PACKED, true>
                   : w4a16_gemm32_split_kernel<WVN, PACKED, false>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(WVN * 2 * 64), lds, stream, W, S, X, Y, N, M);
  return launch_status();
}

template <int WVN, int MT, int NB, bool PACKED>
int launch_gemm32(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                  int K, int M, hipStream_t stream) {
  const size_t lds = gemm32_lds_bytes<WVN, MT>();
  const int gx = (N + 32 * WVN * NB - 1) / (32 * WVN * NB);
  const int gy = (M + 32 * MT - 1) / (32 * MT);
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  const bool svec = !PACKED && (K / kGroup) % 8 == 0 && aligned(S, 16);
  auto kern = svec ? w4a16_gemm32_kernel<WVN, MT, NB, PACKED, true>
                   : w4a16_gemm32_kernel<WVN, MT, NB, PACKED, false>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(WVN * 64), lds, stream, W, S, X, Y, N, K, M);
  return launch_status();
}

}  // namespace

template <bool PACKED>
int launch_prefill32(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                     int K, int M, hipStream_t stream) {
  if (K == kUnit * kGroup) {
    switch (prefill_split_waves(N, M, cu_count(), PACKED)) {
      case 2: return launch_gemm32_split<2, PACKED>(W, S, X, Y, N, M, stream);
      case 4: return launch_gemm32_split<4, PACKED>(W, S, X, Y, N, M, stream);
      default: return launch_gemm32_split<8, PACKED>(W, S, X, Y, N, M, stream);
    }
  }
  return launch_gemm32<8, 1, 1, PACKED>(W, S, X, Y, N, K, M, stream);
}

// Waves per wave set of the K = 1024 split kernel: the narrowest of 2, 4
// and 8 (64, 128 or 256 weight rows per workgroup) whose workgroups fill
// between half and one round of the CUs. M = 512: 512 x 1024 takes 2
// (5.20-5.25 against 5.51-5.56 us for the 64 x 32 unit GEMM), 2048 x 1024
// takes 4 (6.57 against 6.68-6.75 us for the 128 x 32 one), 3584 and 4096
// x 1024 take 8. When none fits, prepacked weights take 4-wave sets (two
// workgroups per CU) from one to 1.5 rounds of those: 6144 x 1024 13.48-13.61
// against 14.37-14.63 us for the unit GEMM; the file layout, whose 4-wave
// sets stage their loads and run one workgroup per CU, keeps the unit GEMM
// (15.9-16.0 against 19.1-19.3 us). 0: the unit GEMM.
int prefill_split_waves(int N, int M, int cus, bool packed) {
  const long long gy = (M + 31) / 32;
  for (int wv = 2; wv <= 8; wv *= 2) {
    const long long wgs = gy * ((N + 32 * wv - 1) / (32 * wv));
    if (2 * wgs >= cus && wgs <= cus) return wv;
  }
  const long long wgs4 = gy * ((N + 127) / 128);
  if (packed && wgs4 >= cus && wgs4 <= 3LL * cus) return 4;
  return 0;
}

int prefill32_regs() { return regs_of(w4a16_gemm32_split_kernel<8, true, false>); }

template int launch_prefill32<true>(const uint8_t*, const uint16_t*, const uint16_t*, uint16_t*,
                                    int, int, int, hipStream_t);
template int launch_prefill32<false>(const uint8_t*, const uint16_t*, const uint16_t*, uint16_t*,
                                     int, int, int, hipStream_t);

}  // namespace cudalm_hip
