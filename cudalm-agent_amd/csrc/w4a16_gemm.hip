// Pipelined prefill-chunk W4A16 GEMM for K = 1024 (MI355X, gfx950). A
// measured alternative to the unit GEMM of w4a16_kernels.hip, selected only
// by CUDALM_W4A16_GEMM_CFG = 50 / 51; it is not faster on the census shapes
// at M = 512 (11-12 us against 10.7 us at 3584x1024), see the numbers below.
//
// Contract (reference: tests/cuda/test_int4_gemv_bf16.cpp:54-69 applied row
// by row; the reference itself runs prefill one token at a time,
// src/runtime/qwen35_generator.cpp:107-125):
//   y[m,n] = bf16_rne( sum_k q[n,k] * f32(s[n,k/128]) * f32(x[m,k]) ).
//
// Work decomposition. A workgroup of WN waves owns an output tile of
// TN = WN * RN * 16 weight rows by TM = RM * 16 activation rows. Wave w owns
// RN 16-row weight tiles and all RM activation tiles, so each weight dword
// is decoded once per workgroup and feeds RM MFMAs, and each activation
// fragment read from LDS feeds RN MFMAs. The 8 groups of the unit run as
// straight-line code: the activations of the next groups arrive through a
// 4-slot register ring (coalesced 64-byte row pieces, put back into MFMA
// operand order by a cross-row lane transpose), each group is staged into
// one of two LDS buffers in pair order with its offset chain, and one
// barrier per group publishes it. Outputs leave through LDS as 16-byte rows.
//
// Per-output operation sequence (identical to every other W4A16 kernel of
// this library, so the bits are the same): per group, tmp = offset chain,
// then four MFMAs of x against the decoded weights seeded with it;
// part = fma(s_g, tmp, part) from 0 in group order; y = bf16_rne(16 * (0 + part)).
//
// Where the time goes (3584x1024x512, 224 workgroups of 4 waves, per-wave
// s_memrealtime probes of the CUDALM_GEMM_PROBE build): about 2 us before
// the first group (the L2 is cold at every dispatch: TCC misses fetch x once
// per XCD, ~10.9 MB per launch), 8 groups of ~0.65-0.75 us each (32 MFMAs,
// ~130 VALU, the staging and one barrier; the MFMAs alone are ~0.3 us at the
// measured 8.75 ns per 16x16x32 MFMA of one wave), and ~0.9 us of output.

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
  g_probe[(blockIdx.x * 8 + wv) * 8 + (k)] = __builtin_amdgcn_s_memrealtime()
#else
#define GEMM_PROBE(k)
#endif

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

// Pipelined variant for K = 1024 (one 8-group unit, the census's common
// case): straight-line code over the 8 groups. Activations of the next
// groups arrive through a 4-slot register ring while the current group is
// computed; each group is staged into one of two LDS buffers (pair order,
// offset chain by the staging wave) and published with one barrier. All
// weights and scales of the unit are requested up front.
template <int WN, int RN, int RM, bool PACKED, bool SVEC>
__global__ __launch_bounds__(WN * 64) void w4a16_gemm_pipe_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int M, int gmb) {
  constexpr int K = kUnit * kGroup, G = kUnit;
  constexpr int TM = RM * 16;
  constexpr int TN = WN * RN * 16;
  constexpr int SPW = (RM + WN - 1) / WN;
  constexpr int RX = 4;  // activation ring (groups)
  // LDS: two group buffers [2][RM][4][64] x 16 B, offsets [2][TM] floats;
  // the output tile [TM][TN + 8] bf16 reuses the group buffers at the end
  extern __shared__ u32x4_t lds[];
  u32x4_t* xs = lds;
  float* offs = reinterpret_cast<float*>(lds + 2 * RM * 4 * 64);

  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, a = lane >> 4;
  const int wv = wave_id();
  GEMM_PROBE(0);
  // XCD-aware numbering (hardware slot L runs on XCD L % 8). When the
  // tile grid splits evenly, XCD x takes a block of gnb/4 weight blocks by
  // gmb/2 activation blocks, which is about the fewest bytes one XCD's L2
  // must pull in; otherwise a contiguous run of the weight-major order.
  const int T = static_cast<int>(gridDim.x);
  const int L = static_cast<int>(blockIdx.x);
  const int gnb = T / gmb;
  int nb, mb;
  if (T % kXcds == 0 && gmb % 2 == 0 && gnb % 4 == 0) {
    const int xcd = L % kXcds, slot = L / kXcds;
    const int mbs = gmb / 2, nbs = gnb / 4;
    const int nn = slot / mbs;
    nb = (xcd >> 1) * nbs + nn;
    mb = (xcd & 1) * mbs + (slot - nn * mbs);
  } else {
    const int lin = (T % kXcds == 0) ? (L % kXcds) * (T / kXcds) + L / kXcds : L;
    nb = lin / gmb;
    mb = lin - nb * gmb;
  }
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
  constexpr int kStep = PACKED ? 1024 : 64;
  const uint16_t* xrow[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s)
    xrow[s] = X + static_cast<size_t>(m0 + min(16 * min(wv + s * WN, RM - 1) + i, mrows - 1)) * K +
              8 * a;

  // load d of lane (i, c) reads row i, 16-byte block 4d + c of the group (the
  // four lanes of a row read 64 contiguous bytes); transpose4() then gives
  // lane (i, a) its own MFMA operand blocks 4a .. 4a+3
  u32x4_t xr[RX][SPW][4];
  auto load_x = [&](u32x4_t (&dst)[SPW][4], int g) {
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
      for (int d = 0; d < 4; ++d)
        dst[s][d] = *reinterpret_cast<const u32x4_t*>(xrow[s] + g * kGroup + 32 * d);
  };
  // the next group in pair order with its offset chains, in registers ...
  struct Staged {
    u32x4_t xa[SPW][4];
    f32x4_t o[SPW];
  };
  auto prepare = [&](Staged& st, const u32x4_t (&src)[SPW][4]) {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      if (wv + s * WN >= RM) continue;  // wave-uniform
      u32x4_t r[4] = {src[s][0], src[s][1], src[s][2], src[s][3]};
      transpose4(r);
#pragma unroll
      for (int d = 0; d < 4; ++d) st.xa[s][d] = pair_order(r[d]);
      st.o[s] = group_offset(st.xa[s]);
    }
  };
  // ... and parked in LDS buffer b
  auto publish = [&](const Staged& st, int b) {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int j = wv + s * WN;
      if (j >= RM) continue;  // wave-uniform
      u32x4_t* blk = xs + ((b * RM + j) * 4) * 64 + lane;
#pragma unroll
      for (int d = 0; d < 4; ++d) blk[d * 64] = st.xa[s][d];
      if (i == 0) *reinterpret_cast<f32x4_t*>(offs + b * TM + 16 * j + 4 * a) = st.o[s];
    }
  };

  // prologue: activations of groups 0 .. 3, then every weight and scale
#pragma unroll
  for (int q = 0; q < RX; ++q) load_x(xr[q], q);
  u32x4_t w[RN][G];
  u32x4_t sc[RN];
#pragma unroll
  for (int gg = 0; gg < G; ++gg)
#pragma unroll
    for (int rn = 0; rn < RN; ++rn)
      w[rn][gg] = *reinterpret_cast<const u32x4_t*>(wl[rn] + static_cast<size_t>(gg) * kStep);
#pragma unroll
  for (int rn = 0; rn < RN; ++rn) {
    if constexpr (PACKED || SVEC) {
      sc[rn] = *reinterpret_cast<const u32x4_t*>(sl[rn]);
    } else {
      const uint16_t* srow = reinterpret_cast<const uint16_t*>(sl[rn]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        sc[rn][q] = static_cast<uint32_t>(srow[2 * q]) | (static_cast<uint32_t>(srow[2 * q + 1]) << 16);
    }
  }
  GEMM_PROBE(1);
  Staged st;
  prepare(st, xr[0]);
  publish(st, 0);
  load_x(xr[0], RX);
  __syncthreads();
  GEMM_PROBE(2);

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t part[RN][RM];
#pragma unroll
  for (int rn = 0; rn < RN; ++rn)
#pragma unroll
    for (int ct = 0; ct < RM; ++ct) part[rn][ct] = zero;
#pragma unroll
  for (int gg = 0; gg < G; ++gg) {
    const int b = gg & 1;
    // the next group's transform and offset chains interleave with this group's MFMAs
    if (gg + 1 < G) {
      prepare(st, xr[(gg + 1) % RX]);
      if (gg + 1 + RX < G) load_x(xr[(gg + 1) % RX], gg + 1 + RX);
    }
    f32x4_t t[RN][RM];
#pragma unroll
    for (int ct = 0; ct < RM; ++ct) {
      const f32x4_t o = *reinterpret_cast<const f32x4_t*>(offs + b * TM + 16 * ct + 4 * a);
#pragma unroll
      for (int rn = 0; rn < RN; ++rn) t[rn][ct] = o;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      u32x4_t xa[RM];
#pragma unroll
      for (int ct = 0; ct < RM; ++ct) xa[ct] = xs[((b * RM + ct) * 4 + d) * 64 + lane];
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
    if (gg == 3) GEMM_PROBE(3);
    if (gg + 1 < G) publish(st, b ^ 1);
    if (gg == 3) GEMM_PROBE(4);
    __syncthreads();
    if (gg == 3) GEMM_PROBE(7);
  }
  GEMM_PROBE(5);

  // outputs: total = 0 + part (the canonical unit sum), then as in the unit kernel
  f32x4_t acc[RN][RM];
#pragma unroll
  for (int rn = 0; rn < RN; ++rn)
#pragma unroll
    for (int ct = 0; ct < RM; ++ct) acc[rn][ct] = zero + part[rn][ct];
  const int n0 = nb * TN;
  const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
  if (vec) {
    constexpr int OP = TN + 8;
    uint16_t* ot = reinterpret_cast<uint16_t*>(lds);
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
    constexpr int PR = TN / 8;
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
}

template <int WN, int RN, int RM, bool PACKED>
int launch_pipe(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N, int K,
                int M, hipStream_t stream) {
  if (K != kUnit * kGroup) return 1;
  constexpr int TN = WN * RN * kTileRows, TM = RM * 16;
  const long long gnb = (N + TN - 1) / TN, gmb = (M + TM - 1) / TM;
  const long long T = gnb * gmb;
  if (T > 0x7FFFFFFFLL) return CUDALM_W4A16_ERANGE;
  const bool svec = !PACKED && aligned(S, 16);
  const size_t xb = static_cast<size_t>(2) * RM * 4 * 64 * 16 + 2 * TM * sizeof(float);
  const size_t ob = static_cast<size_t>(TM) * (TN + 8) * 2;
  const size_t lds = xb > ob ? xb : ob;
  auto kern = svec ? w4a16_gemm_pipe_kernel<WN, RN, RM, PACKED, true>
                   : w4a16_gemm_pipe_kernel<WN, RN, RM, PACKED, false>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(T)), dim3(WN * 64), lds, stream, W, S, X, Y, N,
                     M, static_cast<int>(gmb));
  return launch_status();
}

}  // namespace

template <bool PACKED>
int launch_prefill_group(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                         int K, int M, int cfg, hipStream_t stream) {
  if (cfg < 0) return 1;  // by shape: the unit GEMM of the main kernel file
  switch (cfg) {
    case 50: return launch_pipe<4, 2, 4, PACKED>(W, S, X, Y, N, K, M, stream);  // 128 x 64
    case 51: return launch_pipe<4, 2, 2, PACKED>(W, S, X, Y, N, K, M, stream);  // 128 x 32
    default: return 1;
  }
}

int prefill_group_regs() { return regs_of(w4a16_gemm_pipe_kernel<4, 2, 4, true, false>); }

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
