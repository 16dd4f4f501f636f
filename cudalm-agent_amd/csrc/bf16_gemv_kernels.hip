// bf16 GEMV (the tied LM head) for MI355X (gfx950): kernels and the C-ABI
// launch layer declared in include/cudalm_bf16_gemv.h.
//
// Contract (reference: include/cudalm/kernels/bf16_gemv.h:19-38,
// src/kernels/bf16_gemv.cu:40-129, src/kernels/batch_decode.cu:195-236):
//   y[m,n] = bf16_rne( sum_k f32(W[n,k]) * f32(x[m,k]) ), fp32 accumulation,
//   W bf16 [N, K], x bf16 [M, K], y bf16 [M, N], all row-major.
//
// The weight is read exactly once per launch (for M <= 32 activation rows;
// larger M is split into row chunks that each stream it). bf16 x bf16
// products are exact in fp32, so the matrix cores compute the contraction
// directly: v_mfma_f32_16x16x32_bf16 with activations as the A operand and
// a 16-row weight tile as the B operand. Lane l = 16a + i of MFMA step j in
// unit u holds 16 contiguous bytes of weight row i: k = 256u + 32j + 8a ..
// +7, and reads the same k of its activation row from LDS. Every output is
// one MFMA chain over k in ascending 32-wide steps, so its bits do not
// depend on M, the chunking of M, or which wave or workgroup computed it.
//
// Workload of the LM head (N = 248320, K = 1024, M = 1): 508.6 MB of
// weights, streamed by persistent waves that walk 16-row tiles grid-stride
// in 8 KB units (256 k x 16 rows) and prefetch the next unit while the
// current one is multiplied. Row-major weights are loaded in whole 128 B
// lines and re-laid out through LDS (bf16_unit_load); the tile-major copy
// is already in operand layout.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#include "cudalm_bf16_gemv.h"
#include "hip_common.h"

namespace {

using namespace cudalm_hip;

constexpr int kWaves = 4;              // waves per workgroup
constexpr int kSteps = 8;              // MFMA steps per streamed unit
constexpr int kUnitK = 32 * kSteps;    // k per unit
constexpr int kTile = 16;              // weight rows per tile

struct Bf16Unit {
  u32x4_t w[kSteps];
};

// Row-major weights are loaded coalesced and re-laid out through LDS. The
// MFMA operand layout would make every wave load read 64 B from each of 16
// rows (half lines); instead load q reads whole 128 B lines: rows
// 8 (q & 1) .. +7 of the tile, k quarter q >> 1 of the unit (lane l: row
// 8 (q & 1) + l / 8, k = 256 u + 64 (q >> 1) + 8 (l % 8)). Each quarter (two
// MFMA steps) is written to the wave's staging rows and read back in operand
// layout just before its steps. Rows are kStagePitch bytes apart (128 B of
// data + 16 B) so the 16 rows' operand reads spread over the LDS banks.
// Measured on the LM head (N = 248320, K = 1024, M = 1): 88.4 -> 77.6 us
// (with the sink below).
// Read-only target of a wave's last, unused unit load (both layouts):
// one unit (8 slabs of 1 KB), never written. The loop's loads stay
// unconditional without re-reading a non-temporally loaded unit from HBM.
__device__ __align__(256) uint16_t g_bf16_unit_sink[kSteps * 512];

constexpr int kStagePitch = 144;
constexpr int kStageBytes = kTile * kStagePitch;  // per wave

// Straight-line loads (row and k clamped into the matrix); the k >= K lanes
// are zeroed at use, so a partial last unit or tile needs no branch around
// the loads.
__device__ __forceinline__ void bf16_unit_load(Bf16Unit& v, const uint16_t* __restrict__ W, int N,
                                               int K, int tile, int u, int lane, bool real) {
  const int r = lane >> 3, c = lane & 7;
#pragma unroll
  for (int q = 0; q < kSteps; ++q) {
    const uint16_t* p =
        real ? W + static_cast<size_t>(min(tile * kTile + 8 * (q & 1) + r, N - 1)) * K +
                   min(u * kUnitK + 64 * (q >> 1) + 8 * c, K - 8)
             : g_bf16_unit_sink + q * 512 + lane * 8;
    v.w[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  }
}


// Tile-major layout (cudalm_bf16_repack): the unit u of tile t is 8
// consecutive 1 KB slabs, slab j holding, at byte 16 l, lane l's 16 bytes of
// MFMA step j (row 16 t + l % 16, k = 256 u + 32 j + 8 (l / 16)), so every
// wave-wide load reads 1 KB contiguous. Requires N % 16 == 0, K % 256 == 0.

__device__ __forceinline__ void bf16_unit_load_packed(Bf16Unit& v, const uint16_t* __restrict__ Wp,
                                                      int U, int tile, int u, int lane, bool real) {
  const uint16_t* slab =
      (real ? Wp + (static_cast<size_t>(tile) * U + u) * (kSteps * 512) : g_bf16_unit_sink) + lane * 8;
#pragma unroll
  for (int j = 0; j < kSteps; ++j)
    v.w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(slab + j * 512));
}

// STAGED (row-major loads): v holds the coalesced layout, re-laid out
// through the wave's staging rows `stage` one quarter at a time.
template <int CT, bool STAGED>
__device__ __forceinline__ void bf16_unit_mma(f32x4_t (&acc)[CT], const Bf16Unit& v,
                                              const u32x4_t* const (&xrow)[CT], int u, int K,
                                              int lane, uint8_t* stage) {
  const int i = lane & 15, a = lane >> 4;
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < kSteps; ++j) {
    const int kb = u * kUnitK + 32 * j;  // first k of the step
    u32x4_t w = v.w[j];
    if constexpr (STAGED) {
      if ((j & 1) == 0) {
        // quarter j / 2: loads j and j + 1 (rows 0-7 and 8-15)
#pragma unroll
        for (int q = j; q < j + 2; ++q)
          *reinterpret_cast<u32x4_t*>(stage + (8 * (q & 1) + (lane >> 3)) * kStagePitch +
                                      16 * (lane & 7)) = v.w[q];
        wave_lds_sync();
      }
      w = *reinterpret_cast<const u32x4_t*>(stage + i * kStagePitch + 64 * (j & 1) + 16 * a);
      if (j & 1) wave_lds_sync();  // the quarter is read before the next overwrites it
    }
    const u32x4_t b = kb + 8 * a < K ? w : zero4;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[ct] = mfma16(xrow[ct][(kb >> 3) + a], b, acc[ct]);
  }
}

// Persistent stream kernel. Launch: grid (gx, ceil(M / mc)), 256 threads,
// LDS = stream_lds(K, mc) bytes; chunk y covers activation
// rows [y * mc, y * mc + mc) and mc <= 16 * CT. Requires K % 8 == 0 and
// 16 B aligned W and X bases.
template <int CT, bool PACKED = false>
__global__ __launch_bounds__(kWaves * 64) void bf16_gemv_stream_kernel(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int N, int K, int M, int mc) {
  extern __shared__ u32x4_t xs[];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int i = lane & 15, a = lane >> 4;
  const int U = (K + kUnitK - 1) / kUnitK;
  const int pitch = U * (kUnitK / 8) + 1;  // 16 B blocks per LDS row (padded)
  const int ntiles = (N + kTile - 1) / kTile;
  const int m0 = blockIdx.y * mc;
  const int mrows = min(mc, M - m0);
  const int stride = gridDim.x * kWaves;
  int t = blockIdx.x * kWaves + wave;

  // first unit's weights fly while the activations are staged
  Bf16Unit cur, nxt;
  if constexpr (PACKED)
    bf16_unit_load_packed(cur, W, U, min(t, ntiles - 1), 0, lane, true);
  else
    bf16_unit_load(cur, W, N, K, min(t, ntiles - 1), 0, lane, true);
  const int nb = U * (kUnitK / 8);
  for (int e = threadIdx.x; e < mrows * nb; e += blockDim.x) {
    const int mm = e / nb;
    const int b = e - mm * nb;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (8 * b < K)
      v = *reinterpret_cast<const u32x4_t*>(X + static_cast<size_t>(m0 + mm) * K + 8 * b);
    xs[mm * pitch + b] = v;
  }
  __syncthreads();
  if (t >= ntiles) return;

  // this wave's staging rows (row-major weights), after the activations
  uint8_t* stage =
      reinterpret_cast<uint8_t*>(xs + static_cast<size_t>(mc) * pitch) + wave * kStageBytes;
  const u32x4_t* xrow[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) xrow[ct] = xs + min(ct * 16 + i, mrows - 1) * pitch;

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) acc[ct] = zero;
  int u = 0;
  while (true) {
    int nt = t, nu = u + 1;
    if (nu == U) {
      nu = 0;
      nt = t + stride;
    }
    const bool has_next = nt < ntiles;
    // past the last unit, read the sink unit instead of branching around
    // the loads
    if constexpr (PACKED)
      bf16_unit_load_packed(nxt, W, U, nt, nu, lane, has_next);
    else
      bf16_unit_load(nxt, W, N, K, nt, nu, lane, has_next);
    bf16_unit_mma<CT, !PACKED>(acc, cur, xrow, u, K, lane, stage);
    if (u == U - 1) {
      const int n = t * kTile + i;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = ct * 16 + 4 * a + r;
          if (m < mrows && n < N)
            Y[static_cast<size_t>(m0 + m) * N + n] =
                static_cast<uint16_t>(f32_to_bf16_rne(acc[ct][r]));
        }
        acc[ct] = zero;
      }
    }
    if (!has_next) break;
    cur = nxt;
    t = nt;
    u = nu;
  }
}

// Element-wise fallback for K % 8 != 0, misaligned bases or rows too long
// for LDS (the reference's scalar kernel, bf16_gemv.cu:78-110, serves the
// same cases). One wave per (row n, activation row m): lane-strided fp32
// partial sums, then a butterfly reduction over the wave.
__global__ __launch_bounds__(kWaves * 64) void bf16_gemv_scalar_kernel(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
    int N, int K) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * kWaves + wave_id();
  const int m = blockIdx.y;
  if (n >= N) return;
  const uint16_t* wrow = W + static_cast<size_t>(n) * K;
  const uint16_t* xrow = X + static_cast<size_t>(m) * K;
  float acc = 0.0f;
  for (int k = lane; k < K; k += 64) {
    const float p = bf16_lo(wrow[k]) * bf16_lo(xrow[k]);
    acc = acc + p;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, 64);
  if (lane == 0) Y[static_cast<size_t>(m) * N + n] = static_cast<uint16_t>(f32_to_bf16_rne(acc));
}

// LDS of the stream kernel: mc activation rows, then the staging rows of
// the row-major path (counted for both layouts).
size_t stream_lds(int K, int mc) {
  const int U = (K + kUnitK - 1) / kUnitK;
  return static_cast<size_t>(mc) * (U * (kUnitK / 8) + 1) * 16 + kWaves * kStageBytes;
}

// Activation rows per chunk: up to 32 (two 16-row MFMA column tiles) when
// M > 16, as many as the LDS holds; 0 if not even one row fits.
int stream_rows_per_chunk(int K, int M) {
  int mc = M > 16 ? 32 : M;
  while (mc > 0 && stream_lds(K, mc) > kLdsMax) --mc;
  return mc;
}

// resident workgroups per CU of the persistent bf16 stream kernel
int stream_wgs_per_cu() { return 4; }

template <int CT, bool PACKED = false>
int launch_stream_ct(const uint16_t* W, const uint16_t* X, uint16_t* Y, int N, int K, int M,
                     int mc, hipStream_t stream) {
  const size_t lds = stream_lds(K, mc);
  auto kern = bf16_gemv_stream_kernel<CT, PACKED>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  const int ntiles = (N + kTile - 1) / kTile;
  const int per_cu = static_cast<int>(kLdsMax / lds) < stream_wgs_per_cu()
                         ? static_cast<int>(kLdsMax / lds)
                         : stream_wgs_per_cu();
  // balanced rounds: every wave walks the same number of tiles
  const int cap_waves = cu_count() * (per_cu > 0 ? per_cu : 1) * kWaves;
  const int rounds = (ntiles + cap_waves - 1) / cap_waves;
  const int waves = (ntiles + rounds - 1) / rounds;
  const int gx = (waves + kWaves - 1) / kWaves;
  const int gy = (M + mc - 1) / mc;
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(kWaves * 64), lds, stream, W, X, Y, N, K, M, mc);
  return launch_status();
}

template <bool PACKED = false>
int launch_stream(const uint16_t* W, const uint16_t* X, uint16_t* Y, int N, int K, int M,
                  hipStream_t stream) {
  const int mc = stream_rows_per_chunk(K, M);
  if (mc < 1) return CUDALM_W4A16_EVARIANT;
  if (mc > 16) return launch_stream_ct<2, PACKED>(W, X, Y, N, K, M, mc, stream);
  return launch_stream_ct<1, PACKED>(W, X, Y, N, K, M, mc, stream);
}

// One thread per 16-byte chunk of the tile-major layout.
__global__ __launch_bounds__(256) void bf16_repack_kernel(const uint16_t* __restrict__ W,
                                                          uint16_t* __restrict__ Wp, int K,
                                                          long long nchunks) {
  const long long c = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= nchunks) return;
  const int U = K / kUnitK;
  const int lane = static_cast<int>(c & 63);
  const long long slab = c >> 6;  // (tile * U + u) * kSteps + j
  const int j = static_cast<int>(slab % kSteps);
  const long long tu = slab / kSteps;
  const int u = static_cast<int>(tu % U);
  const long long tile = tu / U;
  const long long row = tile * kTile + (lane & 15);
  const int k = u * kUnitK + 32 * j + 8 * (lane >> 4);
  *reinterpret_cast<u32x4_t*>(Wp + c * 8) =
      *reinterpret_cast<const u32x4_t*>(W + row * K + k);
}

int launch_scalar(const uint16_t* W, const uint16_t* X, uint16_t* Y, int N, int K, int M,
                  hipStream_t stream) {
  if (M > 65535) return CUDALM_W4A16_ERANGE;
  hipLaunchKernelGGL(bf16_gemv_scalar_kernel, dim3((N + kWaves - 1) / kWaves, M),
                     dim3(kWaves * 64), 0, stream, W, X, Y, N, K);
  return launch_status();
}

int check_shape(int N, int K, int M) {
  if (N < 1 || M < 1 || K < 1) return CUDALM_W4A16_EINVAL;
  if (static_cast<long long>(N) + kTile > (1LL << 30) || K > (1 << 28) ||
      static_cast<long long>(M) > 65535LL * 32)
    return CUDALM_W4A16_ERANGE;
  return CUDALM_W4A16_OK;
}

bool stream_ok(const uint16_t* W, const uint16_t* X, int K, int M) {
  return K % 8 == 0 && aligned(W, 16) && aligned(X, 16) && stream_rows_per_chunk(K, M) >= 1;
}

}  // namespace

extern "C" {

int cudalm_bf16_gemv_variant(const uint16_t* weight, const uint16_t* x, uint16_t* y, int N, int K,
                             int M, int variant, hipStream_t stream) {
  if (int rc = check_shape(N, K, M)) return rc;
  if (!weight || !x || !y) return CUDALM_W4A16_ENULL;
  if (!aligned(weight, 2) || !aligned(x, 2) || !aligned(y, 2)) return CUDALM_W4A16_EALIGN;
  const bool vec = stream_ok(weight, x, K, M);
  switch (variant) {
    case CUDALM_BF16_VARIANT_AUTO:
      return vec ? launch_stream(weight, x, y, N, K, M, stream)
                 : launch_scalar(weight, x, y, N, K, M, stream);
    case CUDALM_BF16_VARIANT_STREAM:
      if (!vec) return CUDALM_W4A16_EVARIANT;
      return launch_stream(weight, x, y, N, K, M, stream);
    case CUDALM_BF16_VARIANT_SCALAR:
      return launch_scalar(weight, x, y, N, K, M, stream);
    default:
      return CUDALM_W4A16_EVARIANT;
  }
}

int cudalm_bf16_gemv(const uint16_t* weight, const uint16_t* x, uint16_t* y, int N, int K, int M,
                     hipStream_t stream) {
  return cudalm_bf16_gemv_variant(weight, x, y, N, K, M, CUDALM_BF16_VARIANT_AUTO, stream);
}

size_t cudalm_bf16_packed_bytes(int N, int K) {
  if (N < 1 || K < 1 || N % kTile != 0 || K % kUnitK != 0) return 0;
  return static_cast<size_t>(N) * static_cast<size_t>(K) * 2;
}

int cudalm_bf16_repack(const uint16_t* weight, void* packed, int N, int K, hipStream_t stream) {
  if (int rc = check_shape(N, K, 1)) return rc;
  if (!weight || !packed) return CUDALM_W4A16_ENULL;
  if (N % kTile != 0 || K % kUnitK != 0) return CUDALM_W4A16_EINVAL;
  if (!aligned(weight, 16) || !aligned(packed, 16)) return CUDALM_W4A16_EALIGN;
  const long long nchunks = static_cast<long long>(N) * K / 8;
  hipLaunchKernelGGL(bf16_repack_kernel, dim3(static_cast<unsigned>((nchunks + 255) / 256)),
                     dim3(256), 0, stream, weight, static_cast<uint16_t*>(packed), K, nchunks);
  return launch_status();
}

int cudalm_bf16_gemv_prepacked(const void* packed, const uint16_t* x, uint16_t* y, int N, int K,
                               int M, hipStream_t stream) {
  if (int rc = check_shape(N, K, M)) return rc;
  if (!packed || !x || !y) return CUDALM_W4A16_ENULL;
  if (N % kTile != 0 || K % kUnitK != 0) return CUDALM_W4A16_EINVAL;
  if (!aligned(packed, 16) || !aligned(x, 16) || !aligned(y, 2)) return CUDALM_W4A16_EALIGN;
  if (stream_rows_per_chunk(K, M) < 1) return CUDALM_W4A16_EVARIANT;
  return launch_stream<true>(static_cast<const uint16_t*>(packed), x, y, N, K, M, stream);
}

int cudalm_bf16_gemv_kernel_regs(int variant) {
  switch (variant) {
    case CUDALM_BF16_VARIANT_STREAM: return regs_of(bf16_gemv_stream_kernel<1>);
    case CUDALM_BF16_VARIANT_SCALAR: return regs_of(bf16_gemv_scalar_kernel);
    default: return -1;
  }
}

}  // extern "C"
