// Prefill-chunk W4A16 GEMM (M >= 33) for MI355X (gfx950).
//
// Contract (reference: tests/cuda/test_int4_gemv_bf16.cpp:54-69 applied row
// by row; the reference itself runs prefill one token at a time,
// src/runtime/qwen35_generator.cpp:107-125):
//   y[m,n] = bf16_rne( sum_k q[n,k] * f32(s[n,k/128]) * f32(x[m,k]) ).
//
// Work decomposition. A workgroup of WN waves owns an output tile of
// TN = WN * RN * 16 weight rows by TM = RM * 16 activation rows. Wave w owns
// RN 16-row weight tiles and all RM 16-row activation tiles, so
//   * each weight dword is decoded once per workgroup (by its owner) and
//     feeds RM MFMAs (decode VALU per MFMA = 7 / RM);
//   * each activation fragment read from LDS feeds RN MFMAs (LDS bytes per
//     MFMA = 1 KB / RN).
// K is walked one 128-k quantization group at a time. A group of the tile's
// activations (TM rows x 256 B) is staged into one of two LDS buffers in
// pair order while the previous group is computed; one barrier per group.
// The wave that stages activation tile j also runs that tile's offset chain
// (the four MFMAs of x against -1.5) from the same registers and parks it
// in LDS beside the activations, so an offset chain is run once per
// activation tile and group in the whole workgroup, not once per wave.
//
// Weights and activations arrive through register rings: the weights of
// group g + RW - 1 and the activations of group g + 1 + RX are requested
// while group g is computed.
//
// Per-output operation sequence (identical to the decode kernels): per
// group, tmp = offset chain, then four MFMAs of x against the decoded
// weights in k order seeded with it; part = fma(s_g, tmp, part) from 0 in
// group order within an 8-group unit; total = total + part in unit order
// from 0; y = bf16_rne(16 * total). The bits therefore equal those of every
// other W4A16 kernel of this library.
//
// Workgroups are numbered so that each XCD (workgroups are dealt to the 8
// XCDs round-robin) gets a contiguous run of weight tiles with all of their
// activation blocks: each weight tile is read from HBM into one XCD's L2
// only, and the activations (shared by all weight tiles) are what every
// XCD reads.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "cudalm_w4a16.h"
#include "hip_common.h"
#include "w4a16_device.h"

namespace cudalm_hip {
namespace {

constexpr int kXcds = 8;

#ifdef CUDALM_GEMM_PROBE
// measurement build only: per-wave phase timestamps (s_memrealtime, 100 MHz)
__device__ unsigned long long g_probe[4096 * 8 * 8];
#define GEMM_PROBE(k)                                                           \
  if (lane == 0 && blockIdx.x < 4096)                                           \
  g_probe[(blockIdx.x * 8 + wv + 4 * rep) * 8 + (k)] = __builtin_amdgcn_s_memrealtime()
constexpr int kProbeReps = 2;  // tiles per workgroup, to compare a cold and a warm pass
#else
constexpr int kProbeReps = 1;
#define GEMM_PROBE(k)
#endif

constexpr int kHalf = kUnit / 2;  // groups per staged half unit

// 4 x 4 transpose across the wave's 16-lane rows: afterwards r[d] of row a
// holds what r[a] of row d held. Two v_permlane32_swap and two
// v_permlane16_swap per dword.
__device__ __forceinline__ void transpose4(u32x4_t (&r)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // rows 2, 3 of r0 <-> rows 0, 1 of r2 (and r1 <-> r3)
    auto p02 = __builtin_amdgcn_permlane32_swap(r[0][e], r[2][e], false, false);
    auto p13 = __builtin_amdgcn_permlane32_swap(r[1][e], r[3][e], false, false);
    // rows 1, 3 of r0 <-> rows 0, 2 of r1 (and r2 <-> r3)
    auto p01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
    auto p23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
    r[0][e] = p01[0];
    r[1][e] = p01[1];
    r[2][e] = p23[0];
    r[3][e] = p23[1];
  }
}

// ONE: K fits one 8-group unit (no cross-unit sum is kept).
template <int WN, int RN, int RM, bool PACKED, bool SVEC, bool ONE>
__global__ __launch_bounds__(WN * 64) void w4a16_gemm_lds_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int K, int M, int gmb) {
  constexpr int TM = RM * 16;
  constexpr int TN = WN * RN * 16;
  constexpr int SPW = (RM + WN - 1) / WN;  // activation tiles staged per wave (j = wv + s WN < RM)
  // LDS: activation chunks [RM][kUnit][4][64] x 16 B (chunk (j, g, d) holds
  // lane l's MFMA operand of activation tile j, group g, step d at 16 l, in
  // pair order), then the offset table [kUnit][TM] floats
  extern __shared__ u32x4_t lds[];
  u32x4_t* xs = lds;
  float* offs = reinterpret_cast<float*>(lds + RM * kUnit * 4 * 64);

  const int G = K >> 7;
  const int U = ONE ? 1 : (G + kUnit - 1) / kUnit;
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, a = lane >> 4;
  const int wv = wave_id();
  for (int rep = 0; rep < kProbeReps; ++rep) {
  GEMM_PROBE(0);

  // XCD-aware numbering: hardware slot L runs on XCD L % 8; XCD x gets the
  // contiguous run [x * T / 8, (x + 1) * T / 8) of the (weight block major,
  // activation block minor) order.
  const int T = static_cast<int>(gridDim.x) * kProbeReps;
  const int L = static_cast<int>(blockIdx.x) * kProbeReps + rep;
  const int lin = (T % kXcds == 0) ? (L % kXcds) * (T / kXcds) + L / kXcds : L;
  const int nb = lin / gmb, mb = lin - nb * gmb;
  const int m0 = mb * TM;
  const int mrows = min(TM, M - m0);

  const uint8_t* wl[RN];
  const uint8_t* sl[RN];
  const int first_tile = (nb * WN + wv) * RN;
#pragma unroll
  for (int rn = 0; rn < RN; ++rn) {
    const int rt = min(first_tile + rn, ntiles - 1);
    if constexpr (PACKED) {
      const uint8_t* tile = W + static_cast<size_t>(rt) * packed_tile_bytes(G);
      wl[rn] = tile + lane * 16;
      sl[rn] = tile + static_cast<size_t>(G) * 1024 + i * packed_scale_pitch(G);
    } else {
      const int row = min(rt * kTileRows + i, N - 1);
      wl[rn] = W + static_cast<size_t>(row) * (K >> 1) + a * 16;
      sl[rn] = reinterpret_cast<const uint8_t*>(S + static_cast<size_t>(row) * G);
    }
  }
  constexpr int kStep = PACKED ? 1024 : 64;  // bytes between groups of one lane
  const uint16_t* xrow[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s)
    xrow[s] = X + static_cast<size_t>(m0 + min(16 * min(wv + s * WN, RM - 1) + i, mrows - 1)) * K +
              8 * a;

  // this wave's activations of groups g0 .. g0+3 (indices clamped). Load q
  // of lane (i, c) reads row i, 16-byte block 4q + c of the group, so the
  // four lanes of a row read 64 contiguous bytes; transpose4() then gives
  // lane (i, a) its MFMA operand blocks 4a .. 4a+3.
  auto load_half = [&](u32x4_t (&dst)[SPW][kHalf][4], int g0) {
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
      for (int gg = 0; gg < kHalf; ++gg)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          dst[s][gg][q] = *reinterpret_cast<const u32x4_t*>(xrow[s] + min(g0 + gg, G - 1) * kGroup +
                                                            32 * q);
  };
  // pair order, park in LDS, and the offset chains from the same registers
  auto stage_half = [&](const u32x4_t (&src)[SPW][kHalf][4], int h) {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int j = wv + s * WN;
      if (j >= RM) continue;  // wave-uniform
#pragma unroll
      for (int q = 0; q < kHalf; ++q) {
        const int gg = h * kHalf + q;
        u32x4_t xa[4] = {src[s][q][0], src[s][q][1], src[s][q][2], src[s][q][3]};
        transpose4(xa);
#pragma unroll
        for (int d = 0; d < 4; ++d) xa[d] = pair_order(xa[d]);
        u32x4_t* blk = xs + ((j * kUnit + gg) * 4) * 64 + lane;
#pragma unroll
        for (int d = 0; d < 4; ++d) blk[d * 64] = xa[d];
        const f32x4_t o = group_offset(xa);
        if (i == 0) *reinterpret_cast<f32x4_t*>(offs + gg * TM + 16 * j + 4 * a) = o;
      }
    }
  };

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t acc[RN][RM], part[RN][RM];
#pragma unroll
  for (int rn = 0; rn < RN; ++rn)
#pragma unroll
    for (int ct = 0; ct < RM; ++ct) acc[rn][ct] = zero;

  for (int u = 0; u < U; ++u) {
    const int g0 = u * kUnit;
    const int gn = min(kUnit, G - g0);
    u32x4_t xr[SPW][kHalf][4];
    load_half(xr, g0);
    // the unit's weights and scales (group indices clamped to G - 1)
    u32x4_t w[RN][kUnit];
    u32x4_t sc[RN];
#pragma unroll
    for (int rn = 0; rn < RN; ++rn) {
#pragma unroll
      for (int gg = 0; gg < kUnit; ++gg)
        w[rn][gg] = *reinterpret_cast<const u32x4_t*>(
            wl[rn] + static_cast<size_t>(min(g0 + gg, G - 1)) * kStep);
      if constexpr (PACKED || SVEC) {
        sc[rn] = *reinterpret_cast<const u32x4_t*>(sl[rn] + 2 * g0);
      } else {
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(sl[rn]);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sc[rn][q] = static_cast<uint32_t>(srow[min(g0 + 2 * q, G - 1)]) |
                      (static_cast<uint32_t>(srow[min(g0 + 2 * q + 1, G - 1)]) << 16);
      }
    }
    GEMM_PROBE(1);
    if (u > 0) __syncthreads();  // the previous unit's readers are done
    stage_half(xr, 0);
    if (gn > kHalf) load_half(xr, g0 + kHalf);
    GEMM_PROBE(2);
    __syncthreads();
    GEMM_PROBE(3);

#pragma unroll
    for (int rn = 0; rn < RN; ++rn)
#pragma unroll
      for (int ct = 0; ct < RM; ++ct) part[rn][ct] = zero;
    auto group = [&](int gg) {
      f32x4_t t[RN][RM];
#pragma unroll
      for (int ct = 0; ct < RM; ++ct) {
        const f32x4_t o = *reinterpret_cast<const f32x4_t*>(offs + gg * TM + 16 * ct + 4 * a);
#pragma unroll
        for (int rn = 0; rn < RN; ++rn) t[rn][ct] = o;
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        u32x4_t xa[RM];
#pragma unroll
        for (int ct = 0; ct < RM; ++ct) xa[ct] = xs[((ct * kUnit + gg) * 4 + d) * 64 + lane];
#pragma unroll
        for (int rn = 0; rn < RN; ++rn) {
          const u32x4_t B = decode_nibbles<PACKED>(w[rn][gg][d]);
#pragma unroll
          for (int ct = 0; ct < RM; ++ct) t[rn][ct] = mfma16(xa[ct], B, t[rn][ct]);
        }
      }
#pragma unroll
      for (int rn = 0; rn < RN; ++rn) {
        const float s = half_bits_to_f32((sc[rn][gg >> 1] >> (16 * (gg & 1))) & 0xFFFFu);
#pragma unroll
        for (int ct = 0; ct < RM; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            part[rn][ct][r] = __builtin_fmaf(s, t[rn][ct][r], part[rn][ct][r]);
      }
    };
    // first half while the second half's activations arrive
    if (gn >= kHalf) {
#pragma unroll
      for (int gg = 0; gg < kHalf; ++gg) group(gg);
    } else {
#pragma unroll
      for (int gg = 0; gg < kHalf; ++gg)
        if (gg < gn) group(gg);
    }
    GEMM_PROBE(4);
    if (gn > kHalf) {
      stage_half(xr, 1);
      __syncthreads();
      if (gn == kUnit) {
#pragma unroll
        for (int gg = kHalf; gg < kUnit; ++gg) group(gg);
      } else {
#pragma unroll
        for (int gg = kHalf; gg < kUnit; ++gg)
          if (gg < gn) group(gg);
      }
    }
#pragma unroll
    for (int rn = 0; rn < RN; ++rn)
#pragma unroll
      for (int ct = 0; ct < RM; ++ct) acc[rn][ct] = acc[rn][ct] + part[rn][ct];
  }
  GEMM_PROBE(5);

  // outputs. Lane (i, a) holds rows 4a .. 4a+3 of each activation tile,
  // column i of each weight tile. When rows are 16-byte aligned the tile
  // goes through LDS ([TM][TN + 8] bf16) and leaves as 16-byte row pieces.
  const int n0 = nb * TN;
  const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
  if (vec) {
    constexpr int OP = TN + 8;  // row pitch in bf16 (16 B pad)
    uint16_t* ot = reinterpret_cast<uint16_t*>(lds);
    __syncthreads();  // every wave is done reading activations
#pragma unroll
    for (int rn = 0; rn < RN; ++rn) {
      const int c = (wv * RN + rn) * 16 + i;
#pragma unroll
      for (int ct = 0; ct < RM; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ot[(ct * 16 + 4 * a + r) * OP + c] =
              static_cast<uint16_t>(f32_to_bf16_rne(16.0f * acc[rn][ct][r]));
    }
    __syncthreads();
    constexpr int PR = TN / 8;  // 16-byte pieces per row
    const int ncols = min(TN, N - n0);
    for (int e = threadIdx.x; e < TM * PR; e += WN * 64) {
      const int row = e / PR, pc = e - row * PR;
      if (row < mrows && pc * 8 < ncols)
        *reinterpret_cast<u32x4_t*>(Y + static_cast<size_t>(m0 + row) * N + n0 + pc * 8) =
            *reinterpret_cast<const u32x4_t*>(ot + row * OP + pc * 8);
    }
  } else {
#pragma unroll
    for (int rn = 0; rn < RN; ++rn) {
      const int n = (first_tile + rn) * kTileRows + i;
      if (first_tile + rn >= ntiles || n >= N) continue;
      uint16_t* col = Y + static_cast<size_t>(m0 + 4 * a) * N + n;
#pragma unroll
      for (int ct = 0; ct < RM; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (ct * 16 + 4 * a + r < mrows)
            col[static_cast<size_t>(ct * 16 + r) * N] =
                static_cast<uint16_t>(f32_to_bf16_rne(16.0f * acc[rn][ct][r]));
    }
  }
  GEMM_PROBE(6);
  __syncthreads();
  }
}

template <int WN, int RN, int RM, bool PACKED>
int launch_lds(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N, int K,
               int M, hipStream_t stream) {
  constexpr int TN = WN * RN * kTileRows, TM = RM * 16;
  const long long gnb = (N + TN - 1) / TN, gmb = (M + TM - 1) / TM;
  const long long T = gnb * gmb;
  if (T > 0x7FFFFFFFLL) return CUDALM_W4A16_ERANGE;
  const int G = K / kGroup;
  const bool svec = !PACKED && G % 8 == 0 && aligned(S, 16);
  const size_t lds = static_cast<size_t>(RM) * kUnit * 4 * 64 * 16 + kUnit * TM * sizeof(float);
  const bool one = G <= kUnit;
  auto kern = svec ? (one ? w4a16_gemm_lds_kernel<WN, RN, RM, PACKED, true, true>
                          : w4a16_gemm_lds_kernel<WN, RN, RM, PACKED, true, false>)
                   : (one ? w4a16_gemm_lds_kernel<WN, RN, RM, PACKED, false, true>
                          : w4a16_gemm_lds_kernel<WN, RN, RM, PACKED, false, false>);
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(T / kProbeReps)), dim3(WN * 64), lds, stream, W, S, X, Y,
                     N, K, M, static_cast<int>(gmb));
  return launch_status();
}

}  // namespace

template <bool PACKED>
int launch_prefill_group(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                         int K, int M, int cfg, hipStream_t stream) {
  if (cfg < 0) return 1;  // by shape: the unit GEMM of the main kernel file
  switch (cfg) {
    case 40: return launch_lds<4, 2, 4, PACKED>(W, S, X, Y, N, K, M, stream);  // 128 x 64
    case 41: return launch_lds<4, 1, 4, PACKED>(W, S, X, Y, N, K, M, stream);  // 64 x 64
    case 42: return launch_lds<2, 2, 4, PACKED>(W, S, X, Y, N, K, M, stream);  // 64 x 64, 2 waves
    case 43: return launch_lds<2, 2, 2, PACKED>(W, S, X, Y, N, K, M, stream);  // 64 x 32
    case 44: return launch_lds<4, 2, 2, PACKED>(W, S, X, Y, N, K, M, stream);  // 128 x 32
    case 45: return launch_lds<2, 1, 2, PACKED>(W, S, X, Y, N, K, M, stream);  // 32 x 32
    default: return 1;
  }
}

int prefill_group_regs() { return regs_of(w4a16_gemm_lds_kernel<4, 2, 4, true, false, true>); }

#ifdef CUDALM_GEMM_PROBE
extern "C" int cudalm_gemm_probe_read(void* host, size_t bytes) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_probe), bytes) == hipSuccess ? 0 : -1;
}
#endif

template int launch_prefill_group<true>(const uint8_t*, const uint16_t*, const uint16_t*,
                                        uint16_t*, int, int, int, int, hipStream_t);
template int launch_prefill_group<false>(const uint8_t*, const uint16_t*, const uint16_t*,
                                         uint16_t*, int, int, int, int, hipStream_t);

}  // namespace cudalm_hip
