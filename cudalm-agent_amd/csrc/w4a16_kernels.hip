// W4A16 projection engine for MI355X (gfx950): kernels and the C-ABI launch
// layer declared in include/cudalm_w4a16.h.
//
// Contract (reference: include/cudalm/kernels/int4_gemv_bf16.h:6-9,29-37,
// src/kernels/int4_gemv_bf16.cu:75-170, src/kernels/batch_decode.cu:95-190):
//   y[m,n] = bf16_rne( sum_k q[n,k] * f32(s[n,k/128]) * f32(x[m,k]) ), fp32 acc.
//
// How the contraction maps onto CDNA4 matrix cores
// -------------------------------------------------
// Every kernel computes 16 x 16 output tiles (16 activation rows m x 16
// weight rows n) with v_mfma_f32_16x16x32_bf16, activations as the A
// operand and weights as the B operand. One 128-wide quantization group of
// one 16-row weight tile is a 1 KB slab: lane l = 16a + i holds the 16
// bytes of weight row i that carry k = 32a .. 32a+31 of the group, and each
// of its four dwords feeds one MFMA step (8 k per lane, 32 k per step).
// The lane's activation operand is row i, the same 32 k. After the four
// steps lane l holds the group partial for rows m = 4a .. 4a+3 of column
// n = i, so every lane applies exactly one fp16 group scale.
//
// A weight nibble n (two's complement q) becomes an exact bf16 by bit
// placement: 0x3F80 | ((n ^ 8) << 3) encodes 1 + (q+8)/16 = 1.5 + q/16.
// Two nibbles 16 bits apart become one bf16 pair with one shift and one
// v_bitop3 (8 VALU ops per dword of 8 weights). The constant is removed
// inside the matrix core: a four-step MFMA chain against a constant -1.5
// operand produces -1.5 * sum(x) per row and group, and it seeds the
// accumulator of the weight chain, so
//     tmp = -1.5 * sum_k x  +  sum_k (1.5 + q/16) x  =  (1/16) sum_k q x
// and the per-group epilogue is one fma: acc = fma(s[n,g], tmp, acc); the
// output is bf16_rne(16 * acc). The pair layout produced by the decoder is
// (k, k+4) for k = 0..3 of each 8-k block, so activations sit in LDS in
// that order: [x0 x4 x1 x5 x2 x6 x3 x7].
//
// All kernels run the same per-output operation sequence (same MFMA
// operands in the same slots, same chains, same group order, same
// epilogue), so an output has the same bits whichever kernel, tile shape,
// batch size or weight layout produced it. The tests pin that.
//
// Prepacked ("repacked at load") weight layout, per 16-row tile:
//   [G x 1024 B weights: group g at g*1024, lane l's 16 bytes at 16*l,
//    each little-endian dword of 8 nibbles rotated left by 3 bits]
//   [16 rows x SP B scales: row i at G*1024 + i*SP, fp16 of groups 0..G-1,
//    SP = 16 * ceil(G/8) (zero padded)]
// so one wave load of a group is 1 KB contiguous and one 16-byte load
// brings a lane the scales of 8 consecutive groups. Rows >= N are zero.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#include <type_traits>

#include "cudalm_w4a16.h"
#include "hip_common.h"
#include "w4a16_device.h"

namespace {

using namespace cudalm_hip;


// Activation / output element type of a kernel instance. Both encode a
// weight nibble as an exact value c + q/kUnit in the activation's 16-bit
// format (the nibble in mantissa bits 3..6), cancel c with an MFMA against
// -c, and scale the accumulated sum by kUnit in the epilogue.
struct ActBf16 {
  static constexpr uint32_t kNegOffsetPair = 0xBFC0BFC0u;  // -1.5, -1.5
  static constexpr float kUnit = 16.0f;  // weight element = 1.5 + q / kUnit
  template <bool ROT>
  __device__ static u32x4_t decode(uint32_t w) { return decode_nibbles<ROT>(w); }
  __device__ static f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) { return mfma16(a, b, c); }
  __device__ static uint32_t round(float f) { return f32_to_bf16_rne(f); }
  __device__ static float widen(uint32_t h) { return bf16_lo(h); }
};

// fp16: 1.0 = 0x3C00 with 10 mantissa bits, so q/16 sits at bit 6 and the
// biased nibble (q + 8 = nibble ^ 8) goes to bits 6..9: 0x3C00 | 0x0200 is
// 1.5, and the element is exactly 1.5 + q/16, the bf16 element's value. One
// shift (one rotation from the prepacked form, which is the file dword
// rotated left by 3) and one v_bitop3 per pair: 8 VALU ops per dword.
// Keeping the bias at 1.5 (not 1.0625 + q/128 with the nibble at bits
// 3..6, one op less) keeps the fp32 cancellation of the offset chain as
// small as in bf16: the reference fixtures then stay within 0.5 fp16 ulp.
struct ActF16 {
  static constexpr uint32_t kNegOffsetPair = 0xBE00BE00u;  // -1.5, -1.5
  static constexpr float kUnit = 16.0f;  // weight element = 1.5 + q / kUnit
  template <bool ROT>
  __device__ static u32x4_t decode(uint32_t w) {
    u32x4_t a;
    if constexpr (ROT) {
      a[0] = (rotr(w, 29) & 0x03C003C0u) ^ 0x3E003E00u;
      a[1] = (rotr(w, 1) & 0x03C003C0u) ^ 0x3E003E00u;
      a[2] = (rotr(w, 5) & 0x03C003C0u) ^ 0x3E003E00u;
      a[3] = (rotr(w, 9) & 0x03C003C0u) ^ 0x3E003E00u;
    } else {
      a[0] = ((w << 6) & 0x03C003C0u) ^ 0x3E003E00u;
      a[1] = ((w << 2) & 0x03C003C0u) ^ 0x3E003E00u;
      a[2] = ((w >> 2) & 0x03C003C0u) ^ 0x3E003E00u;
      a[3] = ((w >> 6) & 0x03C003C0u) ^ 0x3E003E00u;
    }
    return a;
  }
  __device__ static f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  // round to nearest even (v_cvt_f16_f32 under the default rounding mode)
  __device__ static uint32_t round(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  __device__ static float widen(uint32_t h) { return half_bits_to_f32(h & 0xFFFFu); }
};

// An activation trait bound to a weight layout: decode() reads file dwords
// (PACKED false) or prepacked, rotated dwords (PACKED true).
template <class Act, bool PACKED>
struct Layout : Act {
  __device__ static u32x4_t decode(uint32_t w) { return Act::template decode<PACKED>(w); }
};

// -1.5 * (sum over the group of this lane-set's activation rows) in the
// activation type Act.
template <class Act>
__device__ __forceinline__ f32x4_t group_offset_t(const u32x4_t (&xa)[4]) {
  const u32x4_t neg = {Act::kNegOffsetPair, Act::kNegOffsetPair, Act::kNegOffsetPair,
                       Act::kNegOffsetPair};
  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t c = Act::mma(xa[0], neg, zero);
  c = Act::mma(xa[1], neg, c);
  c = Act::mma(xa[2], neg, c);
  c = Act::mma(xa[3], neg, c);
  return c;
}

// LDS layout of staged activations. A row holds K/8 16-byte blocks plus
// kXPad pad blocks, so rows start 2 blocks (mod 16) apart, and inside each
// 128-column group the block of lane quarter a, step d (logical block
// 4a + d, columns 32a + 8d ..) sits at slot 4d + a. One ds_read_b128 step
// of a wave then reads 4 adjacent blocks from each of 16 rows: measured
// conflict-free on gfx950 (4 LDS cycles per instruction), where unswizzled
// rows 1 block (mod 16) apart spend half their cycles in bank conflicts.
constexpr int kXPad = 2;
__host__ __device__ constexpr int x_pitch(int kcl) { return (kcl >> 3) + kXPad; }
__device__ __forceinline__ int x_slot(int c) { return (c & ~15) | ((c & 3) << 2) | ((c >> 2) & 3); }

__device__ __forceinline__ void load_group_x(u32x4_t (&xa)[4], const u32x4_t* xgroup, int a) {
#pragma unroll
  for (int d = 0; d < 4; ++d) xa[d] = xgroup[4 * d + a];
}

// scale of group gg (0..7) from 8 packed fp16
__device__ __forceinline__ float unit_scale(u32x4_t sv, int gg) {
  return half_bits_to_f32((sv[gg >> 1] >> (16 * (gg & 1))) & 0xFFFFu);
}

// Stage rows [m0, m0+mrows) x k [k0, k0+kcl) of X into LDS in pair order,
// row pitch `pitch` 16-byte blocks. Thread t moves the 16-byte blocks
// e = t + q * blockDim.x; loads go out in batches of up to 8 per thread
// before any is waited on. A batch is split into stage_load (registers) and
// stage_store (LDS) so that a kernel can issue its first batch ahead of its
// weight loads: memory returns in issue order, so x loaded first is usable
// while the weights are still in flight.
constexpr int kStageBatch = 8;

struct StageBatch {
  u32x4_t v[kStageBatch];
};

// Row and block of the 16-byte blocks a thread stages: block e lies in row
// e / nb at block e % nb, and a thread's blocks are `step` apart, so one
// division per thread starts an incremental walk (step = dm rows + dc blocks)
// instead of a division per block.
struct StageWalk {
  int mm, c, dm, dc, nb;
  __device__ __forceinline__ StageWalk(int e0, int nb_, int step) : nb(nb_) {
    mm = static_cast<int>(static_cast<unsigned>(e0) / static_cast<unsigned>(nb));
    c = e0 - mm * nb;
    dm = static_cast<int>(static_cast<unsigned>(step) / static_cast<unsigned>(nb));
    dc = step - dm * nb;
  }
  __device__ __forceinline__ void next() {
    c += dc;
    mm += dm;
    if (c >= nb) {
      c -= nb;
      ++mm;
    }
  }
};

// Batch b (blocks [b * 8 * blockDim.x, (b + 1) * 8 * blockDim.x)).
__device__ __forceinline__ void stage_load(StageBatch& sb, const uint16_t* __restrict__ X, int K,
                                           int m0, int mrows, int k0, int kcl, int b) {
  const int nb = kcl >> 3;
  const int total = mrows * nb;
  const int step = static_cast<int>(blockDim.x);
  const int first = b * kStageBatch * step;  // uniform
  StageWalk wk(first + static_cast<int>(threadIdx.x), nb, step);
#pragma unroll
  for (int q = 0; q < kStageBatch; ++q) {
    if (first + q * step < total) {  // uniform: whole batches of blocks
      // blocks past the end re-read the last one
      const bool in = first + q * step + static_cast<int>(threadIdx.x) < total;
      const int mm = in ? wk.mm : mrows - 1;
      const int c = in ? wk.c : nb - 1;
      sb.v[q] = *reinterpret_cast<const u32x4_t*>(X + static_cast<size_t>(m0 + mm) * K + k0 + 8 * c);
    }
    wk.next();
  }
}

__device__ __forceinline__ void stage_store(u32x4_t* xs, int pitch, const StageBatch& sb,
                                            int mrows, int kcl, int b) {
  const int nb = kcl >> 3;
  const int total = mrows * nb;
  const int step = static_cast<int>(blockDim.x);
  const int first = b * kStageBatch * step + static_cast<int>(threadIdx.x);
  StageWalk wk(first, nb, step);
#pragma unroll
  for (int q = 0; q < kStageBatch; ++q) {
    if (first + q * step < total) xs[wk.mm * pitch + x_slot(wk.c)] = pair_order(sb.v[q]);
    wk.next();
  }
}

// Batches b0.. to the end.
__device__ __forceinline__ void stage_activations(u32x4_t* xs, int pitch,
                                                  const uint16_t* __restrict__ X, int K, int m0,
                                                  int mrows, int k0, int kcl, int b0 = 0) {
  const int total = mrows * (kcl >> 3);
  const int per_batch = kStageBatch * static_cast<int>(blockDim.x);
  for (int b = b0; b * per_batch < total; ++b) {
    StageBatch sb;
    stage_load(sb, X, K, m0, mrows, k0, kcl, b);
    stage_store(xs, pitch, sb, mrows, kcl, b);
  }
}

// ---------------------------------------------------------------------------
// Stream kernels: M <= 32 (one or two 16-row column tiles, CT), all of x
// resident in LDS; waves stream 16-row weight tiles (grid-stride), fetching
// the next piece while the current one is multiplied. NR = accumulator rows
// per lane that can hold outputs (1 when M == 1, else 4).
// ---------------------------------------------------------------------------

constexpr int kStreamWaves = 4;
constexpr int kMaxProj = CUDALM_W4A16_MAX_PROJ;

// Projections that share one activation matrix, streamed by one launch.
// Tiles are numbered globally; projection j owns tiles
// [tile_end[j-1], tile_end[j]).
// Up to NMAX projections sharing x; tiles are numbered globally in
// projection order. Launches pass the smallest table that holds their
// projections: kernel arguments and the lookup below grow with NMAX (the
// 264-byte table of 8 cost the LM head 0.26 us over the 40-byte one).
template <int NMAX>
struct ProjTab {
  const uint8_t* w[NMAX];
  const uint16_t* s[NMAX];
  uint16_t* y[NMAX];
  int n[NMAX];
  int tile_end[NMAX];
  int count;
  int ntiles;  // tile_end[count - 1]
};
using ProjTable = ProjTab<kMaxProj>;
using ProjOne = ProjTab<1>;
using ProjFour = ProjTab<4>;

// Single-projection launches pass the projection as scalar kernel
// arguments. The library is built with -amdgpu-kernarg-preload-count=16,
// so the first 16 argument dwords arrive preloaded in SGPRs when the
// dispatcher supports it, and the first weight loads do not wait for a
// kernel-argument fetch through the cold scalar cache (a by-value struct
// argument is not preloaded). Census launches: 607 -> 593 us per token
// unfused at M = 1, 495 -> 478 us fused at M = 8.
__device__ __forceinline__ ProjOne make_proj_one(const uint8_t* w, const uint16_t* s, uint16_t* y,
                                                 int n, int ntiles) {
  ProjOne P;
  P.w[0] = w;
  P.s[0] = s;
  P.y[0] = y;
  P.n[0] = n;
  P.tile_end[0] = ntiles;
  P.count = 1;
  P.ntiles = ntiles;
  return P;
}

// The projection that owns tile t. Every field is read at a constant
// offset and chosen with scalar selects, so the kernel-argument loads are
// independent of each other (a data-dependent index would chain three
// kernel-argument round trips ahead of the first weight load; that cost
// 0.35-0.6 us per small launch).

struct ProjView {
  const uint8_t* w;
  const uint16_t* s;
  uint16_t* y;
  int n;
  int begin;  // first global tile of the projection
};

template <int NMAX>
__device__ __forceinline__ ProjView proj_view(const ProjTab<NMAX>& P, int t) {
  ProjView v = {P.w[0], P.s[0], P.y[0], P.n[0], 0};
  if constexpr (NMAX == 1) {
    return v;
  } else {
    if (P.count == 1) return v;
#pragma unroll
    for (int k = 1; k < NMAX; ++k) {
      if (k < P.count && t >= P.tile_end[k - 1]) {
        v.w = P.w[k];
        v.s = P.s[k];
        v.y = P.y[k];
        v.n = P.n[k];
        v.begin = P.tile_end[k - 1];
      }
    }
    return v;
  }
}

// A copy of the first `count` projections of P in a smaller table.
template <int NMAX>
ProjTab<NMAX> shrink_table(const ProjTable& P) {
  ProjTab<NMAX> T = {};
  for (int j = 0; j < P.count && j < NMAX; ++j) {
    T.w[j] = P.w[j];
    T.s[j] = P.s[j];
    T.y[j] = P.y[j];
    T.n[j] = P.n[j];
    T.tile_end[j] = P.tile_end[j];
  }
  T.count = P.count;
  T.ntiles = P.ntiles;
  return T;
}

// Weight bytes of the streaming kernels are read once per launch: loads
// marked non-temporal keep them from displacing the activations and the
// partially written output lines in L2 (LM head 23.8 -> 23.1 us at M = 1,
// 26.9 -> 25.3 us at M = 8, where each tile writes M scattered 32-byte row
// segments that merge in L2 with the neighbouring tiles' segments).
__device__ __forceinline__ u32x4_t load_weights(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

struct StreamUnit {
  u32x4_t w[kUnit];
  u32x4_t s;  // fp16 scales of the unit's 8 groups for this lane's weight row
};

// The fp16 scales of a unit's 8 groups from a file-layout scale row.
template <bool SVEC>
__device__ __forceinline__ void load_unit_scales(StreamUnit& u, const uint16_t* srow, int G, int g0) {
  if constexpr (SVEC) {
    u.s = *reinterpret_cast<const u32x4_t*>(srow + g0);
  } else {
    uint32_t h[kUnit];
#pragma unroll
    for (int gg = 0; gg < kUnit; ++gg) h[gg] = srow[min(g0 + gg, G - 1)];
#pragma unroll
    for (int q = 0; q < 4; ++q) u.s[q] = h[2 * q] | (h[2 * q + 1] << 16);
  }
}

// Loads are unconditional (group indices clamped to G-1) so the compiler's
// memory counters see one straight-line batch per unit and the compute of
// the current unit waits only for its own data.
template <bool PACKED, bool SVEC>
__device__ __forceinline__ void stream_load(StreamUnit& u, const uint8_t* __restrict__ W,
                                            const uint16_t* __restrict__ S, int N, int K, int G,
                                            int rt, int g0, int lane) {
  const int i = lane & 15, a = lane >> 4;
  if constexpr (PACKED) {
    const uint8_t* tile = W + static_cast<size_t>(rt) * packed_tile_bytes(G);
#pragma unroll
    for (int gg = 0; gg < kUnit; ++gg)
      u.w[gg] = load_weights(tile + min(g0 + gg, G - 1) * 1024 + lane * 16);
    u.s = *reinterpret_cast<const u32x4_t*>(tile + static_cast<size_t>(G) * 1024 +
                                            i * packed_scale_pitch(G) + 2 * g0);
  } else {
    const int row = min(rt * kTileRows + i, N - 1);
    const uint8_t* wrow = W + static_cast<size_t>(row) * (K >> 1) + a * 16;
#pragma unroll
    for (int gg = 0; gg < kUnit; ++gg)
      u.w[gg] = load_weights(wrow + min(g0 + gg, G - 1) * 64);
    load_unit_scales<SVEC>(u, S + static_cast<size_t>(row) * G, G, g0);
  }
}

// File-layout units in whole lines (the split kernel at one column tile):
// load q reads rows 16 rt + 2 q and 2 q + 1, 512 contiguous bytes each (the
// unit's 8 groups; lane l: row 2 q + l / 32, byte 16 (l % 32) of the unit)
// instead of 64 B from each of 16 rows, and unit_relayout moves the unit
// into the lane layout through the wave's LDS staging rows. Rows past the
// matrix are clamped to its last row; scales as stream_load.
constexpr int kUnitStagePitch = kUnit * 64 + 16;               // bytes per staged row
constexpr int kUnitStageBytes = kTileRows * kUnitStagePitch;  // per wave

template <bool SVEC, class PT>
__device__ __forceinline__ void stream_load_coal_t(StreamUnit& u, const PT& P, int K, int G, int t,
                                                   int g0, int lane) {
  const ProjView v = proj_view(P, t);
  const int rt = t - v.begin;
  const int c = lane & 31;
  const uint32_t off = static_cast<uint32_t>(min(g0 + (c >> 2), G - 1) * 64 + 16 * (c & 3));
#pragma unroll
  for (int q = 0; q < kUnit; ++q) {
    const int rr = min(rt * kTileRows + 2 * q + (lane >> 5), v.n - 1);
    u.w[q] = load_weights(v.w + static_cast<size_t>(rr) * (K >> 1) + off);
  }
  const int row = min(rt * kTileRows + (lane & 15), v.n - 1);
  load_unit_scales<SVEC>(u, v.s + static_cast<size_t>(row) * G, G, g0);
}

__device__ __forceinline__ void unit_relayout(StreamUnit& out, const StreamUnit& in, uint8_t* stage,
                                              int lane) {
  const int i = lane & 15, a = lane >> 4;
#pragma unroll
  for (int q = 0; q < kUnit; ++q)
    *reinterpret_cast<u32x4_t*>(stage + (2 * q + (lane >> 5)) * kUnitStagePitch + 16 * (lane & 31)) =
        in.w[q];
  wave_lds_sync();
#pragma unroll
  for (int gg = 0; gg < kUnit; ++gg)
    out.w[gg] = *reinterpret_cast<const u32x4_t*>(stage + i * kUnitStagePitch + 64 * gg + 16 * a);
  wave_lds_sync();  // read before the next unit overwrites the rows
  out.s = in.s;
}

template <bool PACKED, bool SVEC, class PT>
__device__ __forceinline__ void stream_load_t(StreamUnit& u, const PT& P, int K, int G,
                                              int t, int g0, int lane) {
  const ProjView v = proj_view(P, t);
  stream_load<PACKED, SVEC>(u, v.w, v.s, v.n, K, G, t - v.begin, g0, lane);
}

// One group of one 16-row weight tile against CT 16-row activation tiles:
// the offset chain comes from the workgroup's table (corr_g), the weight
// chain seeds from it, and the epilogue applies this lane's row scale.
// IOFF: the offset chain is computed here from the group's activation
// fragments (same operands as the workgroup table, so the same bits)
// instead of being read from the LDS table; launches whose waves take at
// most one tile use it to skip the table and its barrier.
template <int NR, int CT, class Act = ActBf16, bool IOFF = false>
__device__ __forceinline__ void group_tmp_x(f32x4_t (&t)[CT], const u32x4_t (&xa)[CT][4],
                                            u32x4_t w, const float* corr_g, int a) {
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    f32x4_t c;
    if constexpr (IOFF) {
      c = group_offset_t<Act>(xa[ct]);
    } else if constexpr (NR == 1) {
      c = f32x4_t{corr_g[ct * 16 + 4 * a], 0.0f, 0.0f, 0.0f};
    } else {
      c = *reinterpret_cast<const f32x4_t*>(corr_g + ct * 16 + 4 * a);
    }
    // the kernels seed rows 1..3 of a lane with 0 when only row 0 is stored
    t[ct] = NR == 1 ? f32x4_t{c[0], 0.0f, 0.0f, 0.0f} : c;
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const u32x4_t B = Act::decode(w[d]);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) t[ct] = Act::mma(xa[ct][d], B, t[ct]);
  }
}

template <int NR, int CT, class Act = ActBf16, bool IOFF = false>
__device__ __forceinline__ void group_tmp(f32x4_t (&t)[CT], const u32x4_t* const (&xrow)[CT],
                                          int g, u32x4_t w, const float* corr_g, int a) {
  u32x4_t xa[CT][4];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) load_group_x(xa[ct], xrow[ct] + g * 16, a);
  group_tmp_x<NR, CT, Act, IOFF>(t, xa, w, corr_g, a);
}

// A lane's activation fragments of group g straight from global memory, in
// the pair order the LDS staging writes (row = min(ct * 16 + i, mrows - 1)).
template <int CT>
__device__ __forceinline__ void load_group_x_global(u32x4_t (&xa)[CT][4],
                                                    const uint16_t* __restrict__ X, int K,
                                                    int mrows, int g, int i, int a) {
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(
        X + static_cast<size_t>(min(ct * 16 + i, mrows - 1)) * K + g * kGroup + 32 * a);
#pragma unroll
    for (int d = 0; d < 4; ++d) xa[ct][d] = pair_order(src[d]);
  }
}

template <int NR, int CT, class Act = ActBf16, bool IOFF = false>
__device__ __forceinline__ void stream_group(f32x4_t (&acc)[CT], const u32x4_t* const (&xrow)[CT],
                                             int g, u32x4_t w, const float* corr_g, float s,
                                             int a) {
  f32x4_t t[CT];
  group_tmp<NR, CT, Act, IOFF>(t, xrow, g, w, corr_g, a);
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[ct][r] = __builtin_fmaf(s, t[ct][r], acc[ct][r]);
}

// Canonical accumulation, shared by every kernel: within one unit of 8
// groups, part = fma(s_g, tmp_g, part) from part = 0 in group order; the
// unit partials are then summed in unit order from 0. The split kernel
// computes unit partials on different waves and reduces them in that order,
// so it produces the same bits as the kernels that walk units serially.

// One unit (up to 8 groups) of one weight tile into `part`.
template <int NR, int CT, class Act = ActBf16, bool IOFF = false>
__device__ __forceinline__ void stream_unit(f32x4_t (&part)[CT], const StreamUnit& cu,
                                            const u32x4_t* const (&xrow)[CT], const float* corr,
                                            int g0, int gn, int a) {
  if (gn == kUnit) {
    // full unit: straight-line, so independent group chains interleave
#pragma unroll
    for (int gg = 0; gg < kUnit; ++gg)
      stream_group<NR, CT, Act, IOFF>(part, xrow, g0 + gg, cu.w[gg], corr + (g0 + gg) * 16 * CT,
                                unit_scale(cu.s, gg), a);
  } else {
#pragma unroll
    for (int gg = 0; gg < kUnit; ++gg)
      if (gg < gn)
        stream_group<NR, CT, Act, IOFF>(part, xrow, g0 + gg, cu.w[gg], corr + (g0 + gg) * 16 * CT,
                                  unit_scale(cu.s, gg), a);
  }
}

// The output of one accumulator: kUnit * total, or, when that is NaN, the
// reference loop's sum for the output (w4a16_ref_dot: infinite and NaN
// activations and overflow keep the reference's semantics).
template <class Act, bool PACKED>
__device__ __forceinline__ float out_value(float total, const uint8_t* w, const uint16_t* s, int K,
                                           int n, const uint16_t* xrow) {
  const float v = Act::kUnit * total;
  if (__builtin_expect(v != v, 0))
    return w4a16_ref_dot<PACKED, std::is_same<Act, ActF16>::value>(w, s, K, n, xrow);
  return v;
}

// Deferred form (the streaming kernels' pipelined loops): the fast values
// are stored and NaNs reported; the kernel re-walks its tiles with fix_tile
// after its loop when any lane saw one, so the reference loop adds no
// registers to the loop.
template <int NR, int CT, class Act, class PT>
__device__ __forceinline__ bool store_tile_fast(const PT& P, int t, const f32x4_t (&total)[CT],
                                                int M, int i, int a) {
  const ProjView v = proj_view(P, t);
  const int Nj = v.n;
  const int n = (t - v.begin) * kTileRows + i;
  if (n >= Nj) return false;
  uint16_t* col = v.y + static_cast<size_t>(4 * a) * Nj + n;
  bool nan = false;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (ct * 16 + 4 * a + r < M) {
        const float f = Act::kUnit * total[ct][r];
        nan = nan || f != f;
        col[static_cast<size_t>(ct * 16 + r) * Nj] = static_cast<uint16_t>(Act::round(f));
      }
    }
  return nan;
}

// Recompute the NaN outputs of tile t (written by store_tile_fast) with the
// reference loop.
template <int NR, int CT, class Act, class PT, bool PACKED>
__device__ __forceinline__ void fix_tile(const PT& P, int t, int M, int i, int a, const uint16_t* X,
                                      int K) {
  const ProjView v = proj_view(P, t);
  const int Nj = v.n;
  const int n = (t - v.begin) * kTileRows + i;
  if (n >= Nj) return;
  uint16_t* col = v.y + static_cast<size_t>(4 * a) * Nj + n;
  for (int ct = 0; ct < CT; ++ct)
    for (int r = 0; r < NR; ++r) {
      const int m = ct * 16 + 4 * a + r;
      if (m >= M) continue;
      uint16_t* yp = col + static_cast<size_t>(ct * 16 + r) * Nj;
      if ((*yp & 0x7FFFu) > 0x7F80u || (Act::kUnit == 16.0f && std::is_same<Act, ActF16>::value &&
                                         (*yp & 0x7FFFu) > 0x7C00u))
        *yp = static_cast<uint16_t>(Act::round(w4a16_ref_dot<PACKED, std::is_same<Act, ActF16>::value>(
            v.w, v.s, K, n, X + static_cast<size_t>(m) * K)));
    }
}

template <int NR, int CT, class Act, class PT, bool PACKED>
__device__ __forceinline__ void store_tile(const PT& P, int t, const f32x4_t (&total)[CT],
                                           int M, int i, int a, const uint16_t* X, int K) {
  const ProjView v = proj_view(P, t);
  const int Nj = v.n;
  const int n = (t - v.begin) * kTileRows + i;
  if (n >= Nj) return;
  // lane's first output row 4a (+16 ct); the rows r of a lane are Nj apart
  uint16_t* col = v.y + static_cast<size_t>(4 * a) * Nj + n;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int m = ct * 16 + 4 * a + r;
      if (m < M)
        col[static_cast<size_t>(ct * 16 + r) * Nj] = static_cast<uint16_t>(Act::round(
            out_value<Act, PACKED>(total[ct][r], v.w, v.s, K, n, X + static_cast<size_t>(m) * K)));
    }
}

// Workgroup prologue of the stream and split kernels: x into LDS (pair
// order), then the -1.5 * sum_k x table per (group, row), which is the same
// for every weight tile (waves split the groups). Returns the LDS offset
// table; xrow[ct] is this lane's activation row of column tile ct.
template <int CT, class Act = ActBf16, bool IOFF = false>
__device__ __forceinline__ float* stream_prologue(u32x4_t* xs, const u32x4_t* (&xrow)[CT],
                                                  const uint16_t* __restrict__ X, int K, int M,
                                                  int wave, int i, int a, const StageBatch& sb0) {
  const int G = K >> 7;
  const int pitch = x_pitch(K);
  float* corr = reinterpret_cast<float*>(xs + M * pitch);
  stage_store(xs, pitch, sb0, M, K, 0);
  stage_activations(xs, pitch, X, K, 0, M, 0, K, 1);
  __syncthreads();
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) xrow[ct] = xs + min(ct * 16 + i, M - 1) * pitch;
  if constexpr (!IOFF) {
    const int nw = static_cast<int>(blockDim.x >> 6);
    for (int g = wave; g < G; g += nw) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        u32x4_t xa[4];
        load_group_x(xa, xrow[ct] + g * 16, a);
        const f32x4_t c = group_offset_t<Act>(xa);
        if (i == 0) *reinterpret_cast<f32x4_t*>(corr + (g * CT + ct) * 16 + 4 * a) = c;
      }
    }
    __syncthreads();
  }
  return corr;
}

// Read-only target of the stream kernel's last, unused piece load: 4 KB of
// piece plus the lane spread, never written. Pointing that load here keeps
// the loop's loads unconditional (a conditional load makes the compiler
// wait for every load in flight at the merge) without re-reading a
// non-temporally loaded piece from HBM; all waves share these lines in L2.
__device__ __align__(256) uint8_t g_piece_sink[4 * 1024 + 64 * 16];

// Piece streaming: the same arithmetic as the stream kernel (the 8-group
// unit partial, then the unit sum), but weights are fetched and consumed in
// pieces of HG groups (HG divides 8), so the compute that trails a wave's
// last load is HG/8 of a unit and the first compute starts after HG groups.
template <int HG>
struct StreamPiece {
  u32x4_t w[HG];
  uint32_t s[(HG + 1) / 2];  // fp16 scales of the HG groups for this lane's weight row
};

// Lane addresses of one tile: its weight bytes and its fp16 scales at group
// 0. Computed once per tile; the pieces add group offsets to them.
struct TileAddr {
  const uint8_t* w;
  const uint8_t* s;
};

template <bool PACKED, class PT>
__device__ __forceinline__ TileAddr tile_addr(const PT& P, int K, int G, int t, int lane) {
  const ProjView v = proj_view(P, t);
  const int rt = t - v.begin;
  const int i = lane & 15, a = lane >> 4;
  if constexpr (PACKED) {
    const uint8_t* tile = v.w + static_cast<size_t>(rt) * packed_tile_bytes(G);
    return {tile + lane * 16, tile + static_cast<size_t>(G) * 1024 + i * packed_scale_pitch(G)};
  } else {
    const int row = min(rt * kTileRows + i, v.n - 1);
    return {v.w + static_cast<size_t>(row) * (K >> 1) + a * 16,
            reinterpret_cast<const uint8_t*>(v.s + static_cast<size_t>(row) * G)};
  }
}

// The fp16 scales of a piece for this lane's weight row (ad.s: the row's
// scales at group 0).
template <int HG, bool PACKED, bool SVEC>
__device__ __forceinline__ void stream_load_scales(StreamPiece<HG>& h, TileAddr ad, int G, int g0) {
  if constexpr (PACKED || SVEC) {
    // packed scale rows are 16 B aligned; SVEC file rows too (G % 8 == 0)
    if constexpr (HG == 4) {
      const uint2 sv = *reinterpret_cast<const uint2*>(ad.s + 2 * g0);
      h.s[0] = sv.x;
      h.s[1] = sv.y;
    } else if constexpr (HG == 1) {
      h.s[0] = *reinterpret_cast<const uint16_t*>(ad.s + 2 * g0);
    } else {
      h.s[0] = *reinterpret_cast<const uint32_t*>(ad.s + 2 * g0);
    }
  } else {
    const uint16_t* srow = reinterpret_cast<const uint16_t*>(ad.s);
    uint32_t v[HG];
#pragma unroll
    for (int gg = 0; gg < HG; ++gg) v[gg] = srow[min(g0 + gg, G - 1)];
#pragma unroll
    for (int q = 0; q < HG / 2; ++q) h.s[q] = v[2 * q] | (v[2 * q + 1] << 16);
    if constexpr (HG == 1) h.s[0] = v[0];
  }
}

// FULL: G is a multiple of HG, so no group index needs clamping.
template <int HG, bool PACKED, bool SVEC, bool FULL>
__device__ __forceinline__ void stream_load_piece(StreamPiece<HG>& h, TileAddr ad, int G, int g0) {
  static_assert(HG == 1 || HG == 2 || HG == 4, "piece of 1, 2 or 4 groups");
  // a piece past a wave's last one is read from g_piece_sink: it must fit
  static_assert(HG * 1024 + 64 * 16 <= sizeof(g_piece_sink), "the sink must hold a whole piece");
  constexpr int kStep = PACKED ? 1024 : 64;  // bytes between groups of one lane
  const uint8_t* wp = ad.w + static_cast<size_t>(g0) * kStep;
#pragma unroll
  for (int gg = 0; gg < HG; ++gg) {
    const int off = FULL ? gg : min(g0 + gg, G - 1) - g0;
    h.w[gg] = load_weights(wp + off * kStep);
  }
  stream_load_scales<HG, PACKED, SVEC>(h, ad, G, g0);
}

// File-layout pieces in whole lines. In the lane layout the MFMA operand
// needs (row 16 rt + i, 16 bytes at 64 g + 16 a), every wave load reads 64 B
// from each of 16 rows. Here a piece of HG groups (2 or 4) is loaded as
// HG * 64 contiguous bytes per row: load q reads rows R q .. R q + R - 1 of
// the tile (R = 16 / HG; lane l: row R q + l / (4 HG), byte 16 (l % 4 HG) of
// the piece), and coal_relayout moves the piece into the lane layout
// through the wave's LDS staging rows. Rows past the matrix are clamped to
// its last row, as in tile_addr.
template <int HG>
struct CoalAddr {
  const uint8_t* w;    // row 16 rt + lane / (4 HG) (clamped) at group 0
  uint32_t d[HG - 1];  // bytes from w to the rows of loads 1 .. HG-1 (clamped)
  const uint8_t* s;    // this lane's scale row (row 16 rt + lane % 16), as tile_addr
};

// bytes per staged row: the piece + 16 (conflict-free writes and reads)
template <int HG>
constexpr int coal_pitch() { return HG * 64 + 16; }
template <int HG>
constexpr int coal_stage_bytes() { return kTileRows * coal_pitch<HG>(); }  // per wave

template <int HG, class PT>
__device__ __forceinline__ CoalAddr<HG> coal_addr(const PT& P, int K, int G, int t, int lane) {
  static_assert(HG == 2 || HG == 4, "whole-line pieces of 2 or 4 groups");
  constexpr int R = kTileRows / HG;
  const ProjView v = proj_view(P, t);
  const int rt = t - v.begin;
  const int r0 = rt * kTileRows + lane / (4 * HG);
  const int rb = min(r0, v.n - 1);
  const uint32_t rowb = static_cast<uint32_t>(K >> 1);
  CoalAddr<HG> c;
  c.w = v.w + static_cast<size_t>(rb) * rowb;
#pragma unroll
  for (int q = 1; q < HG; ++q)
    c.d[q - 1] = static_cast<uint32_t>(min(r0 + R * q, v.n - 1) - rb) * rowb;
  const int row = min(rt * kTileRows + (lane & 15), v.n - 1);
  c.s = reinterpret_cast<const uint8_t*>(v.s + static_cast<size_t>(row) * G);
  return c;
}

template <int HG, bool SVEC, bool FULL>
__device__ __forceinline__ void coal_load_piece(StreamPiece<HG>& h, const CoalAddr<HG>& ad, int G,
                                                int g0, int lane) {
  const int c = lane % (4 * HG);
  const uint32_t off = FULL ? static_cast<uint32_t>(g0 * 64 + 16 * c)
                            : static_cast<uint32_t>(min(g0 + (c >> 2), G - 1) * 64 + 16 * (c & 3));
  h.w[0] = load_weights(ad.w + off);
#pragma unroll
  for (int q = 1; q < HG; ++q) h.w[q] = load_weights(ad.w + ad.d[q - 1] + off);
  stream_load_scales<HG, false, SVEC>(h, TileAddr{ad.w, ad.s}, G, g0);
}

// The loaded piece (coalesced layout) into the lane layout, through this
// wave's staging rows.
template <int HG>
__device__ __forceinline__ void coal_relayout(StreamPiece<HG>& out, const StreamPiece<HG>& in,
                                              uint8_t* stage, int lane) {
  constexpr int R = kTileRows / HG, P = coal_pitch<HG>();
  const int i = lane & 15, a = lane >> 4;
#pragma unroll
  for (int q = 0; q < HG; ++q)
    *reinterpret_cast<u32x4_t*>(stage + (R * q + lane / (4 * HG)) * P + 16 * (lane % (4 * HG))) =
        in.w[q];
  wave_lds_sync();
#pragma unroll
  for (int gg = 0; gg < HG; ++gg)
    out.w[gg] = *reinterpret_cast<const u32x4_t*>(stage + i * P + 64 * gg + 16 * a);
  wave_lds_sync();  // read before the next piece overwrites the rows
#pragma unroll
  for (int q = 0; q < (HG + 1) / 2; ++q) out.s[q] = in.s[q];
}

template <int HG, int NR, int CT, class Act, bool FULL, bool IOFF = false>
__device__ __forceinline__ void stream_piece(f32x4_t (&part)[CT], const StreamPiece<HG>& h,
                                             const u32x4_t* const (&xrow)[CT], const float* corr,
                                             int g0, int gn, int a) {
#pragma unroll
  for (int gg = 0; gg < HG; ++gg) {
    if (FULL || gg < gn)
      stream_group<NR, CT, Act, IOFF>(part, xrow, g0 + gg, h.w[gg], corr + (g0 + gg) * 16 * CT,
                                half_bits_to_f32((h.s[gg >> 1] >> (16 * (gg & 1))) & 0xFFFFu), a);
  }
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act, int HG, bool FULL, int WV, bool IOFF,
          class PT>
__device__ __forceinline__ void stream_piece_body(
    const PT& P, const uint16_t* __restrict__ X, int K, int M, int pwg, int t_static) {
  extern __shared__ u32x4_t xs[];
  constexpr int PPU = kUnit / HG;  // pieces per 8-group unit
  const int G = K >> 7;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int i = lane & 15, a = lane >> 4;
  const int H = (G + HG - 1) / HG;  // pieces per tile
  // Workgroups [0, pwg) are persistent and stride over tiles [0, t_static);
  // the rest take one tile per wave of [t_static, ntiles). Most of those are
  // resident from the start (the CUs hold more workgroups than the
  // persistent ones) and add loads in flight during the start-up ramp; the
  // others are placed as workgroups retire.
  const bool persistent = static_cast<int>(blockIdx.x) < pwg;
  const int ntiles = persistent ? t_static : P.ntiles;
  const int stride = persistent ? pwg * WV : ntiles;
  int t = persistent ? blockIdx.x * WV + wave : t_static + (blockIdx.x - pwg) * WV + wave;
  const bool active = t < ntiles;

  // File-layout weights of one column tile are loaded in whole lines and
  // re-laid out through per-wave LDS staging rows after the offset table.
  constexpr bool COAL = !PACKED && HG == 4 && CT == 1;
  using Addr = typename std::conditional<COAL, CoalAddr<HG>, TileAddr>::type;
  auto addr_of = [&](int tt) -> Addr {
    if constexpr (COAL)
      return coal_addr<HG>(P, K, G, tt, lane);
    else
      return tile_addr<PACKED>(P, K, G, tt, lane);
  };
  auto load_piece = [&](StreamPiece<HG>& b, const Addr& ad, int g0) {
    if constexpr (COAL)
      coal_load_piece<HG, SVEC, FULL>(b, ad, G, g0, lane);
    else
      stream_load_piece<HG, PACKED, SVEC, FULL>(b, ad, G, g0);
  };
  uint8_t* stage = reinterpret_cast<uint8_t*>(xs) + static_cast<size_t>(M) * x_pitch(K) * 16 +
                   static_cast<size_t>(G) * 64 * CT + wave * coal_stage_bytes<HG>();

  // x's first batch, then the first piece's weights, fly together
  StageBatch sb0;
  stage_load(sb0, X, K, 0, M, 0, K, 0);
  StreamPiece<HG> bufA, bufB;
  Addr acur = addr_of(min(t, ntiles - 1));
  load_piece(bufA, acur, 0);
  const u32x4_t* xrow[CT];
  const float* corr = stream_prologue<CT, Act, IOFF>(xs, xrow, X, K, M, wave, i, a, sb0);
  if (!active) return;

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t part[CT], total[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) part[ct] = total[ct] = zero;
  // the finished tile's sums, stored at the next step (after its wait)
  f32x4_t done[CT];
  int done_t = -1;
  int h = 0;
  // One piece. Loads and stores share one in-order memory counter: the
  // step waits for all of its memory operations first (the current piece),
  // then stores the tile finished in the previous step, then issues the
  // next piece's loads, so no wait ever covers a store issued just before
  // it. The two piece buffers alternate (two steps per loop turn).
  const int t_first = t;
  bool nan_seen = false;
  auto step = [&](const StreamPiece<HG>& cur, StreamPiece<HG>& nxt) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt at their maxima
    if (done_t >= 0) {
      nan_seen |= store_tile_fast<NR, CT, Act, PT>(P, done_t, done, M, i, a);
      done_t = -1;
    }
    int nt = t, nh = h + 1;
    if (nh == H) {
      nh = 0;
      nt = t + stride;
    }
    const bool has_next = nt < ntiles;
    Addr anx = acur;
    if (has_next && nh == 0) anx = addr_of(nt);
    // past the last piece, load from the sink instead of branching around
    // the loads (the scales re-read the current tile's, cached)
    if (!has_next) {
      anx.w = g_piece_sink + lane * 16;
      if constexpr (COAL)
#pragma unroll
        for (int q = 0; q < HG - 1; ++q) anx.d[q] = 0;
    }
    load_piece(nxt, anx, (has_next ? nh : 0) * HG);
    const int g0 = h * HG;
    if constexpr (COAL) {
      StreamPiece<HG> lay;
      coal_relayout(lay, cur, stage, lane);
      stream_piece<HG, NR, CT, Layout<Act, PACKED>, FULL, IOFF>(part, lay, xrow, corr, g0,
                                                               min(HG, G - g0), a);
    } else {
      stream_piece<HG, NR, CT, Layout<Act, PACKED>, FULL, IOFF>(part, cur, xrow, corr, g0,
                                                               min(HG, G - g0), a);
    }
    // an 8-group unit ends after its last piece or at the tile's last piece
    if ((h % PPU) == PPU - 1 || h == H - 1) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        total[ct] = total[ct] + part[ct];
        part[ct] = zero;
      }
    }
    if (h == H - 1) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        done[ct] = total[ct];
        total[ct] = zero;
      }
      done_t = t;
    }
    acur = anx;
    t = nt;
    h = nh;
    return has_next;
  };
  while (step(bufA, bufB) && step(bufB, bufA)) {
  }
  if (done_t >= 0) nan_seen |= store_tile_fast<NR, CT, Act, PT>(P, done_t, done, M, i, a);
  if (__builtin_expect(__builtin_amdgcn_ballot_w64(nan_seen) != 0, 0)) {
    // a NaN sum (infinite or NaN activations, overflow): those outputs are
    // recomputed by the reference loop, which keeps its semantics
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete
    for (int tt = t_first; tt < ntiles; tt += stride)
      fix_tile<NR, CT, Act, PT, PACKED>(P, tt, M, i, a, X, K);
  }
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act = ActBf16, int HG = 4, bool FULL = true,
          int WV = kStreamWaves, bool IOFF = false, class PT = ProjTable>
__global__ __launch_bounds__(WV * 64) void w4a16_stream_piece_kernel(
    const PT P, const uint16_t* __restrict__ X, int K, int M, int pwg, int t_static) {
  stream_piece_body<PACKED, NR, SVEC, CT, Act, HG, FULL, WV, IOFF, PT>(P, X, K, M, pwg, t_static);
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act, int HG, bool FULL, int WV, bool IOFF>
__global__ __launch_bounds__(WV * 64) void w4a16_stream_piece_one_kernel(
    const uint8_t* w, const uint16_t* s, uint16_t* y, int n, int ntiles,
    const uint16_t* __restrict__ X, int K, int M, int pwg, int t_static) {
  stream_piece_body<PACKED, NR, SVEC, CT, Act, HG, FULL, WV, IOFF, ProjOne>(
      make_proj_one(w, s, y, n, ntiles), X, K, M, pwg, t_static);
}

// Split kernel: few weight tiles, several units per tile (K >= 2048). A
// workgroup takes TPR = max(1, 4/U) tiles; its waves compute the unit
// partials of those tiles side by side, park them in LDS, and the unit
// partials of each tile are summed in unit order. Same bits as the stream
// kernel; shorter latency when tiles alone cannot fill the machine.
template <bool PACKED, int NR, bool SVEC, int CT, class Act, class PT>
__device__ __forceinline__ void split_body(const PT& P, const uint16_t* __restrict__ X, int K,
                                           int M) {
  extern __shared__ u32x4_t xs[];
  const int G = K >> 7;
  const int pitch = x_pitch(K);
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int i = lane & 15, a = lane >> 4;
  const int ntiles = P.ntiles;
  const int U = (G + kUnit - 1) / kUnit;
  const int TPR = U >= kStreamWaves ? 1 : kStreamWaves / U;
  const int nslots = TPR * U;
  const int t0 = blockIdx.x * TPR;
  // slot partials after the offset table: [nslots][CT][64 lanes] f32x4
  f32x4_t* slots = reinterpret_cast<f32x4_t*>(
      reinterpret_cast<float*>(xs + M * pitch) + G * 16 * CT);
  // file-layout weights of one column tile: whole-line loads, re-laid out
  // through per-wave staging rows after the slots
  constexpr bool COAL = !PACKED && CT == 1;
  uint8_t* stage = reinterpret_cast<uint8_t*>(slots + static_cast<size_t>(nslots) * CT * 64) +
                   wave * kUnitStageBytes;
  StreamUnit cur;
  auto load_unit = [&](int sl) {
    const int t = min(t0 + sl / U, ntiles - 1), g0 = (sl % U) * kUnit;
    if constexpr (COAL)
      stream_load_coal_t<SVEC>(cur, P, K, G, t, g0, lane);
    else
      stream_load_t<PACKED, SVEC>(cur, P, K, G, t, g0, lane);
  };

  // x's first batch, then this wave's first slot loads, fly together
  StageBatch sb0;
  stage_load(sb0, X, K, 0, M, 0, K, 0);
  load_unit(min(wave, nslots - 1));
  const u32x4_t* xrow[CT];
  const float* corr = stream_prologue<CT, Act, true>(xs, xrow, X, K, M, wave, i, a, sb0);

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int sl = wave; sl < nslots; sl += kStreamWaves) {
    if (sl != wave) load_unit(sl);
    f32x4_t part[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) part[ct] = zero;
    const int g0 = (sl % U) * kUnit;
    if constexpr (COAL) {
      StreamUnit lay;
      unit_relayout(lay, cur, stage, lane);
      stream_unit<NR, CT, Layout<Act, PACKED>, true>(part, lay, xrow, corr, g0, min(kUnit, G - g0), a);
    } else {
      stream_unit<NR, CT, Layout<Act, PACKED>, true>(part, cur, xrow, corr, g0, min(kUnit, G - g0), a);
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) slots[(sl * CT + ct) * 64 + lane] = part[ct];
  }
  __syncthreads();
  if (wave < TPR && t0 + wave < ntiles) {
    f32x4_t total[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      total[ct] = zero;
      for (int u = 0; u < U; ++u) total[ct] = total[ct] + slots[((wave * U + u) * CT + ct) * 64 + lane];
    }
    store_tile<NR, CT, Act, PT, PACKED>(P, t0 + wave, total, M, i, a, X, K);
  }
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act = ActBf16, class PT = ProjTable>
__global__ __launch_bounds__(kStreamWaves * 64) void w4a16_split_kernel(
    const PT P, const uint16_t* __restrict__ X, int K, int M) {
  split_body<PACKED, NR, SVEC, CT, Act, PT>(P, X, K, M);
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act>
__global__ __launch_bounds__(kStreamWaves * 64) void w4a16_split_one_kernel(
    const uint8_t* w, const uint16_t* s, uint16_t* y, int n, int ntiles,
    const uint16_t* __restrict__ X, int K, int M) {
  split_body<PACKED, NR, SVEC, CT, Act, ProjOne>(make_proj_one(w, s, y, n, ntiles), X, K, M);
}

// ---------------------------------------------------------------------------
// SwiGLU epilogue: the MLP's gate and up projections share x, and the down
// projection consumes silu(gate) * up (reference: src/runtime/
// qwen35_deltanet.cpp:236-251, src/kernels/qwen35_kernels.cu:458-476).
// ---------------------------------------------------------------------------

// Element-wise silu(gate) * up over n values; 8 per thread (16 B vectors
// when the three bases are 16 B aligned, element-wise otherwise).
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gate,
                                                       const uint16_t* __restrict__ up,
                                                       uint16_t* __restrict__ y, size_t n,
                                                       int vec) {
  const size_t e0 = (static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (e0 >= n) return;
  if (vec && e0 + 8 <= n) {
    const u32x4_t g = *reinterpret_cast<const u32x4_t*>(gate + e0);
    const u32x4_t u = *reinterpret_cast<const u32x4_t*>(up + e0);
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = silu_mul_bits(g[q] & 0xFFFFu, u[q] & 0xFFFFu) |
             (silu_mul_bits(g[q] >> 16, u[q] >> 16) << 16);
    *reinterpret_cast<u32x4_t*>(y + e0) = o;
  } else {
    const size_t e1 = e0 + 8 < n ? e0 + 8 : n;
    for (size_t e = e0; e < e1; ++e) y[e] = static_cast<uint16_t>(silu_mul_bits(gate[e], up[e]));
  }
}

// gate and up W4A16 projections of the same x (P.count == 2, equal N, gate
// first) with the SwiGLU epilogue, one launch. Work is split like the split
// kernel: a workgroup takes TPR = max(1, 4 / (2U)) row tiles; each tile's
// 2U unit partials (U of gate, then U of up) are computed on separate waves
// and summed in unit order per projection, so gate and up carry exactly the
// bits of their single-projection calls before the epilogue. Activation
// rows are processed in chunks of mc <= 16 * CT rows (blockIdx.y).
template <bool PACKED, int NR, bool SVEC, int CT>
__global__ __launch_bounds__(kStreamWaves * 64) void w4a16_swiglu_kernel(
    const ProjTable P, const uint16_t* __restrict__ X, int K, int M, int mc) {
  extern __shared__ u32x4_t xs[];
  const int G = K >> 7;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int i = lane & 15, a = lane >> 4;
  const int nt = P.tile_end[0];  // row tiles per projection
  const int N = P.n[0];
  const int U = (G + kUnit - 1) / kUnit;
  const int TPR = 2 * U >= kStreamWaves ? 1 : kStreamWaves / (2 * U);
  const int nslots = TPR * 2 * U;
  const int t0 = blockIdx.x * TPR;
  const int m0 = blockIdx.y * mc;
  const int mrows = min(mc, M - m0);
  const int pitch = x_pitch(K);
  f32x4_t* slots = reinterpret_cast<f32x4_t*>(
      reinterpret_cast<float*>(xs + mrows * pitch) + G * 16 * CT);

  // slot sl -> (row tile t0 + sl / 2U, projection (sl % 2U) / U, unit sl % U)
  auto slot_load = [&](StreamUnit& u, int sl) {
    const int tf = min(t0 + sl / (2 * U), nt - 1);
    const int r = sl % (2 * U);
    stream_load_t<PACKED, SVEC>(u, P, K, G, (r / U) * nt + tf, (r % U) * kUnit, lane);
  };
  StageBatch sb0;
  stage_load(sb0, X + static_cast<size_t>(m0) * K, K, 0, mrows, 0, K, 0);
  StreamUnit cur;
  slot_load(cur, min(wave, nslots - 1));
  const u32x4_t* xrow[CT];
  const float* corr =
      stream_prologue<CT, ActBf16, true>(xs, xrow, X + static_cast<size_t>(m0) * K, K, mrows, wave, i,
                                          a, sb0);

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int sl = wave; sl < nslots; sl += kStreamWaves) {
    if (sl != wave) slot_load(cur, sl);
    f32x4_t part[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) part[ct] = zero;
    const int g0 = (sl % U) * kUnit;
    stream_unit<NR, CT, Layout<ActBf16, PACKED>, true>(part, cur, xrow, corr, g0, min(kUnit, G - g0),
                                                      a);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) slots[(sl * CT + ct) * 64 + lane] = part[ct];
  }
  __syncthreads();
  if (wave < TPR && t0 + wave < nt) {
    const int n = (t0 + wave) * kTileRows + i;
    const int base = wave * 2 * U;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      f32x4_t tg = zero, tu = zero;
      for (int u = 0; u < U; ++u) tg = tg + slots[((base + u) * CT + ct) * 64 + lane];
      for (int u = 0; u < U; ++u) tu = tu + slots[((base + U + u) * CT + ct) * 64 + lane];
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int m = ct * 16 + 4 * a + r;
        if (m < mrows && n < N)
          P.y[0][static_cast<size_t>(m0 + m) * N + n] = static_cast<uint16_t>(silu_mul_bits(
              f32_to_bf16_rne(out_value<ActBf16, PACKED>(tg[r], P.w[0], P.s[0], K, n,
                                                         X + static_cast<size_t>(m0 + m) * K)),
              f32_to_bf16_rne(out_value<ActBf16, PACKED>(tu[r], P.w[1], P.s[1], K, n,
                                                         X + static_cast<size_t>(m0 + m) * K))));
      }
    }
  }
}

// Piece split kernel: the split kernel with pieces of HG groups per wave,
// so a unit's groups are multiplied on PPU = 8/HG waves side by side. The
// wave holding a unit's first piece runs its fma chain from 0; the waves
// holding the later pieces park each group's tmp and scale, and the
// reducing wave continues the unit's chain over them in group order before
// the unit sum: the same fma sequence as a serial walk, so the same bits.
// NP = 1: the tiles of every projection in P, stored as outputs. NP = 2:
// SwiGLU; P holds gate then up with equal N, row tile t is gate tile t and
// up tile nt + t, and the output is silu(gate) * up on the bf16-rounded
// projections (blockIdx.y walks chunks of mc activation rows).

template <bool PACKED, int NR, bool SVEC, int CT, class Act, int HG, int WV, int NP, bool DX,
          class PT>
__device__ __forceinline__ void split_piece_body(
    const PT& P, const uint16_t* __restrict__ X, int K, int M, int mc) {
  extern __shared__ u32x4_t xs[];
  constexpr int PPU = kUnit / HG;
  const int G = K >> 7;
  const int pitch = x_pitch(K);
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int i = lane & 15, a = lane >> 4;
  const int nt = NP == 1 ? P.ntiles : P.tile_end[0];  // row tiles
  const int U = (G + kUnit - 1) / kUnit;
  const int H = (G + HG - 1) / HG;  // pieces of a tile that hold groups
  const int SP = U * PPU;           // piece slots of one projection's tile
  const int ST = NP * SP;           // piece slots of a row tile
  const int TPR = ST >= WV ? 1 : WV / ST;
  const int nslots = TPR * ST;
  const int t0 = blockIdx.x * TPR;
  const int m0 = NP == 1 ? 0 : blockIdx.y * mc;
  const int mrows = NP == 1 ? M : min(mc, M - m0);
  const uint16_t* Xc = X + static_cast<size_t>(m0) * K;
  // after x (none with DX): heads [TPR*NP*U][CT][64] f32x4, then the later
  // pieces' tmps [TPR*NP*U][PPU-1][HG][CT][64] f32x4, then their scales
  // [TPR*NP*U][PPU-1][HG][16]
  f32x4_t* heads = reinterpret_cast<f32x4_t*>(xs + (DX ? 0 : mrows * pitch));
  f32x4_t* tmps = heads + TPR * NP * U * CT * 64;
  float* scs = reinterpret_cast<float*>(tmps + TPR * NP * U * (PPU - 1) * HG * CT * 64);

  StageBatch sb0;
  if constexpr (!DX) stage_load(sb0, Xc, K, 0, mrows, 0, K, 0);
  // file-layout pieces of 2 or 4 groups at one column tile: whole-line
  // loads into raw, re-laid out into cur through per-wave staging rows
  // after the scales
  constexpr bool COAL = !PACKED && CT == 1 && (HG == 2 || HG == 4);
  uint8_t* stage = reinterpret_cast<uint8_t*>(scs + TPR * NP * U * (PPU - 1) * HG * 16) +
                   wave * coal_stage_bytes<COAL ? HG : 2>();
  StreamPiece<HG> cur, raw;
  // DX: the piece's activation fragments, loaded by the wave itself
  u32x4_t xg[DX ? HG : 1][CT][4];
  // slot sl -> row tile t0 + sl / ST, projection (sl % ST) / SP, piece sl % SP
  auto load_slot = [&](int sl) {
    const int tf = min(t0 + sl / ST, nt - 1);
    const int pj = (sl % ST) / SP;
    const int h = min(sl % SP, H - 1);
    if constexpr (DX) {
#pragma unroll
      for (int gg = 0; gg < HG; ++gg)
        load_group_x_global<CT>(xg[DX ? gg : 0], Xc, K, mrows, min(h * HG + gg, G - 1), i, a);
    }
    if constexpr (COAL)
      coal_load_piece<HG, SVEC, false>(raw, coal_addr<HG>(P, K, G, pj * nt + tf, lane), G, h * HG,
                                       lane);
    else
      stream_load_piece<HG, PACKED, SVEC, false>(cur, tile_addr<PACKED>(P, K, G, pj * nt + tf, lane),
                                                 G, h * HG);
  };
  load_slot(min(wave, nslots - 1));
  const u32x4_t* xrow[CT];
  const float* corr = nullptr;
  if constexpr (!DX) corr = stream_prologue<CT, Act, true>(xs, xrow, Xc, K, mrows, wave, i, a, sb0);

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int sl = wave; sl < nslots; sl += WV) {
    if (sl != wave) load_slot(sl);
    if constexpr (COAL) coal_relayout<HG>(cur, raw, stage, lane);
    const int tu = sl / SP;  // (row tile, projection) pair, local
    const int h = sl % SP;
    const int u = h / PPU, pp = h % PPU;
    const int g0 = h * HG;
    if (pp == 0) {
      f32x4_t part[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) part[ct] = zero;
      if constexpr (DX) {
#pragma unroll
        for (int gg = 0; gg < HG; ++gg) {
          if (gg < G - g0) {
            f32x4_t t[CT];
            group_tmp_x<NR, CT, Layout<Act, PACKED>, true>(t, xg[DX ? gg : 0], cur.w[gg], corr, a);
            const float sc = half_bits_to_f32((cur.s[gg >> 1] >> (16 * (gg & 1))) & 0xFFFFu);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
              for (int r = 0; r < NR; ++r) part[ct][r] = __builtin_fmaf(sc, t[ct][r], part[ct][r]);
          }
        }
      } else {
        stream_piece<HG, NR, CT, Layout<Act, PACKED>, false, true>(part, cur, xrow, corr, g0,
                                                                    min(HG, G - g0), a);
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) heads[((tu * U + u) * CT + ct) * 64 + lane] = part[ct];
    } else if (g0 < G) {
      const int base = ((tu * U + u) * (PPU - 1) + pp - 1) * HG;
#pragma unroll
      for (int gg = 0; gg < HG; ++gg) {
        if (g0 + gg < G) {
          f32x4_t t[CT];
          if constexpr (DX)
            group_tmp_x<NR, CT, Layout<Act, PACKED>, true>(t, xg[DX ? gg : 0], cur.w[gg], corr, a);
          else
            group_tmp<NR, CT, Layout<Act, PACKED>, true>(t, xrow, g0 + gg, cur.w[gg], corr, a);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) tmps[((base + gg) * CT + ct) * 64 + lane] = t[ct];
          if (a == 0)
            scs[(base + gg) * 16 + i] =
                half_bits_to_f32((cur.s[gg >> 1] >> (16 * (gg & 1))) & 0xFFFFu);
        }
      }
    }
  }
  __syncthreads();
  if (wave < TPR && t0 + wave < nt) {
    f32x4_t total[NP][CT];
#pragma unroll
    for (int pj = 0; pj < NP; ++pj) {
      const int tu = wave * NP + pj;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) total[pj][ct] = zero;
      for (int u = 0; u < U; ++u) {
        // every parked tmp and scale of the unit first (the reads go out
        // together), then the fma chain in group order
        constexpr int NPK = (PPU - 1) * HG;
        f32x4_t p[CT];
        f32x4_t tv[NPK > 0 ? NPK : 1][CT];
        float sv[NPK > 0 ? NPK : 1];
        const int gbase = u * PPU * HG;  // first group of the unit
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) p[ct] = heads[((tu * U + u) * CT + ct) * 64 + lane];
#pragma unroll
        for (int q = 0; q < NPK; ++q) {
          const int base = (tu * U + u) * NPK + q;
          if (gbase + HG + q < G) {
            sv[q] = scs[base * 16 + i];
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) tv[q][ct] = tmps[(base * CT + ct) * 64 + lane];
          }
        }
#pragma unroll
        for (int q = 0; q < NPK; ++q) {
          if (gbase + HG + q < G) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
              for (int r = 0; r < NR; ++r) p[ct][r] = __builtin_fmaf(sv[q], tv[q][ct][r], p[ct][r]);
          }
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) total[pj][ct] = total[pj][ct] + p[ct];
      }
    }
    if constexpr (NP == 1) {
      store_tile<NR, CT, Act, PT, PACKED>(P, t0 + wave, total[0], M, i, a, X, K);
    } else {
      const int N = P.n[0];
      const int n = (t0 + wave) * kTileRows + i;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int m = ct * 16 + 4 * a + r;
          if (m < mrows && n < N)
            P.y[0][static_cast<size_t>(m0 + m) * N + n] = static_cast<uint16_t>(silu_mul_bits(
                f32_to_bf16_rne(out_value<ActBf16, PACKED>(total[0][ct][r], P.w[0], P.s[0], K, n,
                                                           Xc + static_cast<size_t>(m) * K)),
                f32_to_bf16_rne(out_value<ActBf16, PACKED>(total[NP - 1][ct][r], P.w[NP - 1],
                                                           P.s[NP - 1], K, n,
                                                           Xc + static_cast<size_t>(m) * K))));
        }
    }
  }
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act, int HG, int WV, int NP = 1,
          bool DX = false, class PT = ProjTable>
__global__ __launch_bounds__(WV * 64) void w4a16_split_piece_kernel(
    const PT P, const uint16_t* __restrict__ X, int K, int M, int mc) {
  split_piece_body<PACKED, NR, SVEC, CT, Act, HG, WV, NP, DX, PT>(P, X, K, M, mc);
}

// Up to four projections sharing x, as scalar arguments: the first 16
// dwords (weights, tile ends, count, x, K, M) are what the first loads of a
// prepacked launch need; scales, outputs and row counts follow.
template <bool PACKED, int NR, bool SVEC, int CT, class Act, int HG, int WV, bool DX>
__global__ __launch_bounds__(WV * 64) void w4a16_split_piece_four_kernel(
    const uint8_t* w0, const uint8_t* w1, const uint8_t* w2, const uint8_t* w3, int te0, int te1,
    int te2, int count, const uint16_t* __restrict__ X, int K, int M, const uint16_t* s0,
    const uint16_t* s1, const uint16_t* s2, const uint16_t* s3, uint16_t* y0, uint16_t* y1,
    uint16_t* y2, uint16_t* y3, int n0, int n1, int n2, int n3, int ntiles) {
  ProjFour P;
  P.w[0] = w0;
  P.w[1] = w1;
  P.w[2] = w2;
  P.w[3] = w3;
  P.s[0] = s0;
  P.s[1] = s1;
  P.s[2] = s2;
  P.s[3] = s3;
  P.y[0] = y0;
  P.y[1] = y1;
  P.y[2] = y2;
  P.y[3] = y3;
  P.n[0] = n0;
  P.n[1] = n1;
  P.n[2] = n2;
  P.n[3] = n3;
  P.tile_end[0] = te0;
  P.tile_end[1] = te1;
  P.tile_end[2] = te2;
  P.tile_end[3] = ntiles;
  P.count = count;
  P.ntiles = ntiles;
  split_piece_body<PACKED, NR, SVEC, CT, Act, HG, WV, 1, DX, ProjFour>(P, X, K, M, M);
}

// The SwiGLU pair (NP = 2: gate, then up, sharing x; act into y0), as
// scalar arguments, the first 16 dwords being what the first loads need.
template <bool PACKED, int NR, bool SVEC, int CT, int HG, int WV, bool DX>
__global__ __launch_bounds__(WV * 64) void w4a16_split_piece_pair_kernel(
    const uint8_t* w0, const uint8_t* w1, int nt, int count, const uint16_t* __restrict__ X, int K,
    int M, int mc, const uint16_t* s0, const uint16_t* s1, uint16_t* y0, uint16_t* y1, int n0,
    int n1, int ntiles) {
  ProjTab<2> P;
  P.w[0] = w0;
  P.w[1] = w1;
  P.s[0] = s0;
  P.s[1] = s1;
  P.y[0] = y0;
  P.y[1] = y1;
  P.n[0] = n0;
  P.n[1] = n1;
  P.tile_end[0] = nt;
  P.tile_end[1] = ntiles;
  P.count = count;
  P.ntiles = ntiles;
  split_piece_body<PACKED, NR, SVEC, CT, ActBf16, HG, WV, 2, DX, ProjTab<2>>(P, X, K, M, mc);
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act, int HG, int WV, bool DX>
__global__ __launch_bounds__(WV * 64) void w4a16_split_piece_one_kernel(
    const uint8_t* w, const uint16_t* s, uint16_t* y, int n, int ntiles,
    const uint16_t* __restrict__ X, int K, int M) {
  split_piece_body<PACKED, NR, SVEC, CT, Act, HG, WV, 1, DX, ProjOne>(
      make_proj_one(w, s, y, n, ntiles), X, K, M, M);
}

// ---------------------------------------------------------------------------
// Tile kernel: any M. A workgroup of WN x WM waves owns a (WN*RB*16) x
// (WM*CT*16) output tile (n x m); K is walked in chunks of GPC groups whose
// activations are staged in LDS; each wave preloads the chunk's weights.
// ---------------------------------------------------------------------------

template <int RB, int CT, int WN, int WM, int GPC, bool PACKED>
__global__ __launch_bounds__(WN * WM * 64) void w4a16_tile_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int K, int M) {
  extern __shared__ u32x4_t xs[];
  constexpr int CM = WM * CT * 16;
  constexpr int KC = GPC * kGroup;
  constexpr int pitch = x_pitch(KC);
  const int G = K >> 7;
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int wn = wave % WN, wm = wave / WN;
  const int i = lane & 15, a = lane >> 4;
  const int m0 = blockIdx.y * CM;
  const int mrows = min(CM, M - m0);

  int rt[RB];
  bool rt_ok[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = (blockIdx.x * WN + wn) * RB + rb;
    rt_ok[rb] = r < ntiles;
    rt[rb] = min(r, ntiles - 1);
  }
  int xr[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) xr[ct] = min(wm * CT * 16 + ct * 16 + i, mrows - 1) * pitch;

  static_assert(kUnit % GPC == 0, "chunks must not straddle an 8-group unit");
  // acc: the current unit's partial; total: unit partials summed in order
  f32x4_t acc[RB][CT], total[RB][CT];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rb][ct] = total[rb][ct] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int g0 = 0; g0 < G; g0 += GPC) {
    const int ng = min(GPC, G - g0);
    // this chunk's weight and scale loads fly during staging
    u32x4_t w[GPC][RB];
    float s[GPC][RB];
#pragma unroll
    for (int gl = 0; gl < GPC; ++gl) {
      if (gl < ng) {
        const int g = g0 + gl;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          if constexpr (PACKED) {
            const uint8_t* tile = W + static_cast<size_t>(rt[rb]) * packed_tile_bytes(G);
            w[gl][rb] = *reinterpret_cast<const u32x4_t*>(tile + g * 1024 + lane * 16);
            s[gl][rb] = half_bits_to_f32(*reinterpret_cast<const uint16_t*>(
                tile + static_cast<size_t>(G) * 1024 + i * packed_scale_pitch(G) + 2 * g));
          } else {
            const int row = min(rt[rb] * kTileRows + i, N - 1);
            w[gl][rb] = *reinterpret_cast<const u32x4_t*>(
                W + static_cast<size_t>(row) * (K >> 1) + g * 64 + a * 16);
            s[gl][rb] = half_bits_to_f32(S[static_cast<size_t>(row) * G + g]);
          }
        }
      }
    }
    __syncthreads();  // the previous chunk's LDS reads are done
    stage_activations(xs, pitch, X, K, m0, mrows, g0 * kGroup, ng * kGroup);
    __syncthreads();

#pragma unroll
    for (int gl = 0; gl < GPC; ++gl) {
      if (gl < ng) {
        u32x4_t xa[CT][4];
        f32x4_t tp[RB][CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          load_group_x(xa[ct], xs + xr[ct] + gl * 16, a);
          const f32x4_t corr = group_offset(xa[ct]);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) tp[rb][ct] = corr;
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            const u32x4_t B = decode_nibbles<PACKED>(w[gl][rb][d]);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) tp[rb][ct] = mfma16(xa[ct][d], B, tp[rb][ct]);
          }
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[rb][ct][r] = __builtin_fmaf(s[gl][rb], tp[rb][ct][r], acc[rb][ct][r]);
      }
    }
    if ((g0 + ng) % kUnit == 0 || g0 + ng == G) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          total[rb][ct] = total[rb][ct] + acc[rb][ct];
          acc[rb][ct] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
  }

#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    if (!rt_ok[rb]) continue;
    const int n = rt[rb] * kTileRows + i;
    if (n >= N) continue;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ml = wm * CT * 16 + ct * 16 + 4 * a + r;
        if (ml < mrows)
          Y[static_cast<size_t>(m0 + ml) * N + n] = static_cast<uint16_t>(
              f32_to_bf16_rne(out_value<ActBf16, PACKED>(total[rb][ct][r], W, S, K, n,
                                                         X + static_cast<size_t>(m0 + ml) * K)));
      }
  }
}

// ---------------------------------------------------------------------------
// Unit GEMM kernel (prefill chunks): a k-slice of WV waves owns
// TN = WV * RB * 16 weight rows and TM = CT * 16 activation rows. K is walked
// one 8-group unit (1024 k) at a time: the unit's activations are staged
// once into LDS (pair order), the slice computes the unit's offset table
// once (waves split the chains), and every weight is decoded once, by the
// wave that owns its rows, and feeds CT MFMA column tiles. Weights of a unit
// are fetched up front (while the activations are staged). The per-output
// operation sequence is the stream kernel's, so the bits are the same.
//
// KS > 1 k-slices split the units of the same output tile: slice s takes
// units s, s + KS, ... with its own LDS buffers, keeps each unit partial,
// and at the end the partials meet in LDS and are summed in unit order, so
// the bits do not depend on KS. This serves few-tile, long-K shapes
// (N = 1024, K = 2048 / 3584), where one slice would walk every unit alone.
// ---------------------------------------------------------------------------

constexpr int kSliceMaxUnits = 4;  // units per k-slice kept as partials (KS > 1)

template <int RB, int CT, int WV, bool PACKED, bool SVEC, int KS = 1, bool IOFF = false>
__global__ __launch_bounds__(WV * KS * 64) void w4a16_gemm_unit_kernel(
    const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, int N, int K, int M) {
  constexpr int NT = WV * 64;  // threads of one k-slice
  constexpr int TM = CT * 16;
  constexpr int PB = x_pitch(kUnit * kGroup);  // LDS row pitch in 16-byte blocks (padded)
  constexpr int NBLK = TM * kUnit * 16;  // 16-byte x blocks per unit
  static_assert(NBLK % NT == 0, "staging must cover the tile exactly");
  constexpr int BPT = NBLK / NT;  // x blocks staged per thread per unit
  constexpr int XB = TM * PB;     // 16-byte blocks of one slice's x buffer
  constexpr int NPART = KS == 1 ? 1 : kSliceMaxUnits;
  extern __shared__ u32x4_t lds[];  // [KS][TM][PB] x, then [KS] offset tables

  const int G = K >> 7;
  const int U = (G + kUnit - 1) / kUnit;
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int lane = threadIdx.x & 63;
  const int slice = KS == 1 ? 0 : wave_id() / WV;
  const int wave = wave_id() - slice * WV;  // wave within the slice
  const int tid = static_cast<int>(threadIdx.x) - slice * NT;
  const int i = lane & 15, a = lane >> 4;
  const int m0 = blockIdx.y * TM;
  const int mrows = min(TM, M - m0);
  u32x4_t* xs = lds + slice * XB;
  float* corr = reinterpret_cast<float*>(lds + KS * XB) + slice * (kUnit * CT * 16);

  int rt[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) rt[rb] = min((blockIdx.x * WV + wave) * RB + rb, ntiles - 1);
  const bool any_ok = (blockIdx.x * WV + wave) * RB < ntiles;

  // lane addresses of each owned tile at group 0
  const uint8_t* wbase[RB];
  const uint8_t* sbase[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    if constexpr (PACKED) {
      const uint8_t* tile = W + static_cast<size_t>(rt[rb]) * packed_tile_bytes(G);
      wbase[rb] = tile + lane * 16;
      sbase[rb] = tile + static_cast<size_t>(G) * 1024 + i * packed_scale_pitch(G);
    } else {
      const int row = min(rt[rb] * kTileRows + i, N - 1);
      wbase[rb] = W + static_cast<size_t>(row) * (K >> 1) + a * 16;
      sbase[rb] = reinterpret_cast<const uint8_t*>(S + static_cast<size_t>(row) * G);
    }
  }
  constexpr int kStep = PACKED ? 1024 : 64;  // bytes between groups of one lane

  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // KS == 1: the running unit sum; KS > 1: this slice's unit partials
  f32x4_t acc[NPART][RB][CT];
#pragma unroll
  for (int q = 0; q < NPART; ++q)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[q][rb][ct] = zero;

  const int iters = (U + KS - 1) / KS;
  for (int it = 0; it < iters; ++it) {
    const int u = it * KS + slice;
    const int uc = min(u, U - 1);  // a slice past the last unit re-reads it and skips the math
    const int g0 = uc * kUnit;
    const int gn = u < U ? min(kUnit, G - g0) : 0;
    // the unit's activations first: they are staged and feed the offset
    // table before any weight is used, and loads return in issue order
    constexpr int RS = NT / (kUnit * 16);
    static_assert(NT % (kUnit * 16) == 0, "a thread keeps one block column");
    const int b = tid & (kUnit * 16 - 1);  // thread tid stages block b of rows tid / 128 + q * RS
    const int r0 = tid / (kUnit * 16);
    u32x4_t v[BPT];
    {
      const uint16_t* xcol = X + static_cast<size_t>(m0) * K + min(g0 * kGroup + 8 * b, K - 8);
#pragma unroll
      for (int q = 0; q < BPT; ++q)
        v[q] = *reinterpret_cast<const u32x4_t*>(
            xcol + static_cast<size_t>(min(r0 + q * RS, mrows - 1)) * K);
    }
    // then this unit's weights and scales (group indices clamped to G - 1)
    u32x4_t w[RB][kUnit];
    uint32_t sc[RB][kUnit / 2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int gg = 0; gg < kUnit; ++gg)
        w[rb][gg] = *reinterpret_cast<const u32x4_t*>(
            wbase[rb] + static_cast<size_t>(min(g0 + gg, G - 1)) * kStep);
      if constexpr (PACKED || SVEC) {
        const u32x4_t sv = *reinterpret_cast<const u32x4_t*>(sbase[rb] + 2 * g0);
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[rb][q] = sv[q];
      } else {
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(sbase[rb]);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sc[rb][q] = static_cast<uint32_t>(srow[min(g0 + 2 * q, G - 1)]) |
                      (static_cast<uint32_t>(srow[min(g0 + 2 * q + 1, G - 1)]) << 16);
      }
    }
    if (it > 0) __syncthreads();  // previous unit's readers are done
    {
      u32x4_t* xdst = xs + r0 * PB + x_slot(b);
#pragma unroll
      for (int q = 0; q < BPT; ++q) xdst[q * RS * PB] = pair_order(v[q]);
    }
    __syncthreads();
    // offset table of the unit: chains (group, column tile) split over waves
    // (IOFF: each wave runs the chains of its own groups inline instead, the
    // same operands, and the table and its barrier are skipped)
    if constexpr (!IOFF) {
      for (int c = wave; c < kUnit * CT; c += WV) {
        const int gg = c / CT, ct = c - gg * CT;
        u32x4_t xa[4];
        load_group_x(xa, xs + (ct * 16 + i) * PB + gg * 16, a);
        const f32x4_t o = group_offset(xa);
        if (i == 0) *reinterpret_cast<f32x4_t*>(corr + c * 16 + 4 * a) = o;
      }
      __syncthreads();
    }
    if (!any_ok) continue;

    f32x4_t part[RB][CT];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) part[rb][ct] = zero;
    // one group: offset-seeded weight chains, then the scale fma into part
    auto group = [&](int gg) {
      u32x4_t xa[CT][4];
      f32x4_t t[RB][CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        load_group_x(xa[ct], xs + (ct * 16 + i) * PB + gg * 16, a);
        const f32x4_t o = IOFF ? group_offset(xa[ct])
                               : *reinterpret_cast<const f32x4_t*>(corr + (gg * CT + ct) * 16 + 4 * a);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) t[rb][ct] = o;
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const u32x4_t B = decode_nibbles<PACKED>(w[rb][gg][d]);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) t[rb][ct] = mfma16(xa[ct][d], B, t[rb][ct]);
        }
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const float s = half_bits_to_f32((sc[rb][gg >> 1] >> (16 * (gg & 1))) & 0xFFFFu);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            part[rb][ct][r] = __builtin_fmaf(s, t[rb][ct][r], part[rb][ct][r]);
      }
    };
    if (gn == kUnit) {
      // full unit: straight-line, so independent group chains interleave
#pragma unroll
      for (int gg = 0; gg < kUnit; ++gg) group(gg);
    } else {
#pragma unroll
      for (int gg = 0; gg < kUnit; ++gg)
        if (gg < gn) group(gg);
    }
    if constexpr (KS == 1) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[0][rb][ct] = acc[0][rb][ct] + part[rb][ct];
    } else {
#pragma unroll
      for (int q = 0; q < NPART; ++q)
        if (q == it)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[q][rb][ct] = part[rb][ct];
    }
  }

  f32x4_t total[RB][CT];
  if constexpr (KS == 1) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) total[rb][ct] = acc[0][rb][ct];
  } else {
    // unit partials meet in LDS (over the x buffers): slot [u][wave][rb][ct][lane]
    __syncthreads();
    f32x4_t* slots = reinterpret_cast<f32x4_t*>(lds);
    if (any_ok) {
#pragma unroll
      for (int q = 0; q < NPART; ++q) {
        const int u = q * KS + slice;
        if (q < iters && u < U)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
              slots[(((u * WV + wave) * RB + rb) * CT + ct) * 64 + lane] = acc[q][rb][ct];
      }
    }
    __syncthreads();
    if (slice != 0) return;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        total[rb][ct] = zero;
        for (int u = 0; u < U; ++u)
          total[rb][ct] = total[rb][ct] + slots[(((u * WV + wave) * RB + rb) * CT + ct) * 64 + lane];
      }
  }
  if (!any_ok) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int n = ((blockIdx.x * WV + wave) * RB + rb) * kTileRows + i;
    if (n >= N) continue;
    uint16_t* col = Y + static_cast<size_t>(m0 + 4 * a) * N + n;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (ct * 16 + 4 * a + r < mrows)
          col[static_cast<size_t>(ct * 16 + r) * N] = static_cast<uint16_t>(f32_to_bf16_rne(
              out_value<ActBf16, PACKED>(total[rb][ct][r], W, S, K, n,
                                         X + static_cast<size_t>(m0 + ct * 16 + 4 * a + r) * K)));
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

template <class Act>
__global__ __launch_bounds__(256) void w4a16_bytewise_kernel(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ Sb,
    const uint8_t* __restrict__ Xb, uint8_t* __restrict__ Yb, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave_id();
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
    const float x0 = Act::widen(load_u16_bytes(xrow + 4 * b));
    const float x1 = Act::widen(load_u16_bytes(xrow + 4 * b + 2));
    acc += (static_cast<float>(lo) * s) * x0;
    acc += (static_cast<float>(hi) * s) * x1;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) {
    const uint32_t y = Act::round(acc);
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
    const float e0 = (bf16_lo(pairs[p]) - 1.5f) * 16.0f;               // element k0 + p
    const float e1 = (bf16_lo(pairs[p] >> 16) - 1.5f) * 16.0f;         // element k0 + p + 4
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
// Load-time repack: file layout -> prepacked tiles (layout at the top of the
// file). One thread per 16-byte unit of the output.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void w4a16_repack_kernel(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ Sb, uint8_t* __restrict__ P, int N,
    int K) {
  const int G = K >> 7;
  const int SP = packed_scale_pitch(G);
  const size_t units_per_tile = packed_tile_bytes(G) / 16;
  const size_t nunits = static_cast<size_t>((N + 15) / 16) * units_per_tile;
  const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= nunits) return;
  const int rt = static_cast<int>(idx / units_per_tile);
  const int j = static_cast<int>(idx - static_cast<size_t>(rt) * units_per_tile);
  uint8_t out[16];
  if (j < G * 64) {
    const int g = j >> 6, l = j & 63;
    const int n = rt * 16 + (l & 15);
    const int a = l >> 4;
    for (int b = 0; b < 16; ++b)
      out[b] = (n < N) ? W[static_cast<size_t>(n) * (K >> 1) + g * 64 + a * 16 + b] : 0;
  } else {
    const int jj = j - G * 64;
    const int row = jj / (SP / 16), u = jj - row * (SP / 16);
    const int n = rt * 16 + row;
    for (int q = 0; q < 8; ++q) {
      const int g = 8 * u + q;
      const bool ok = n < N && g < G;
      const size_t so = (static_cast<size_t>(n) * G + g) * 2;
      out[2 * q] = ok ? Sb[so] : 0;
      out[2 * q + 1] = ok ? Sb[so + 1] : 0;
    }
  }
  u32x4_t v;
  for (int q = 0; q < 4; ++q) {
    v[q] = static_cast<uint32_t>(out[4 * q]) | (static_cast<uint32_t>(out[4 * q + 1]) << 8) |
           (static_cast<uint32_t>(out[4 * q + 2]) << 16) |
           (static_cast<uint32_t>(out[4 * q + 3]) << 24);
    if (j < G * 64) v[q] = prepack_dword(v[q]);
  }
  reinterpret_cast<u32x4_t*>(P)[idx] = v;
}

// ---------------------------------------------------------------------------
// host launch layer
// ---------------------------------------------------------------------------



int check_shape(int N, int K, int M) {
  if (N < 1 || M < 1 || K <= 0 || K % kGroup != 0) return CUDALM_W4A16_EINVAL;
  // 32-bit tile/group indices inside the kernels
  if (static_cast<long long>(N) + 16 > (1LL << 30) || K > (1 << 24) ||
      static_cast<long long>(M) > 65535LL * 128)
    return CUDALM_W4A16_ERANGE;
  return CUDALM_W4A16_OK;
}


size_t stream_lds_bytes(int K, int M) {
  const int CT = M > 16 ? 2 : 1;
  return static_cast<size_t>(M) * x_pitch(K) * 16 + static_cast<size_t>(K / kGroup) * 64 * CT;
}

// LDS of the stream kernel: x and the offset table, plus the file-layout
// staging rows at one column tile.
size_t stream_kernel_lds(int K, int M, bool packed) {
  const int WV = M > 16 ? 8 : kStreamWaves;
  return stream_lds_bytes(K, M) +
         (!packed && M <= 16 ? static_cast<size_t>(WV) * coal_stage_bytes<4>() : 0);
}

bool stream_fits(int K, int M, bool packed) {
  return M <= 32 && stream_kernel_lds(K, M, packed) <= kLdsMax;
}

int split_tiles_per_round(int K) {
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  return U >= kStreamWaves ? 1 : kStreamWaves / U;
}

size_t split_lds_bytes(int K, int M) {
  const int CT = M > 16 ? 2 : 1;
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  return stream_lds_bytes(K, M) +
         static_cast<size_t>(split_tiles_per_round(K)) * U * CT * 64 * 16;
}

// LDS of the split kernel: split_lds_bytes plus the file-layout staging
// rows at one column tile.
size_t split_kernel_lds(int K, int M, bool packed) {
  return split_lds_bytes(K, M) +
         (!packed && M <= 16 ? static_cast<size_t>(kStreamWaves) * kUnitStageBytes : 0);
}

bool split_fits(int K, int M, bool packed) {
  return M <= 32 && split_kernel_lds(K, M, packed) <= kLdsMax;
}

// Resident workgroups per CU of the persistent stream kernels: 3 of the
// 4-wave one-column-tile kernel, 2 of the 8-wave two-column-tile kernel
// (measured best on the LM head). A variant streaming two adjacent weight
// tiles per wave for M > 16 (each activation fragment read from LDS feeds
// both tiles' MFMAs) holds ~230 VGPRs, so 8 waves per CU; with the
// conflict-free activation layout the one-tile kernel's 16 waves per CU are
// 0.8-1.6 us faster at M = 17..32 on the LM head, so the variant was removed.
constexpr int kStreamWgsPerCu = 3;
constexpr int kStreamWideWgsPerCu = 2;

template <bool PACKED, int NR, bool SVEC, int CT, class Act = ActBf16>
int launch_stream_t(const ProjTable& P, const uint16_t* X, int K, int M, hipStream_t stream) {
  // Two column tiles (M > 16) hold up to 64 KB of x per workgroup, so at
  // most two workgroups fit a CU: 8-wave workgroups keep 16 waves resident
  // (measured 3.5 us faster than 4-wave ones on the M = 32 LM head).
  constexpr int WV = CT == 2 ? 8 : kStreamWaves;
  // file-layout weights at one column tile: the staging rows after the table
  const size_t lds = stream_kernel_lds(K, M, PACKED);
  const int ntiles = P.ntiles;
  int per_cu = CT == 2 ? kStreamWideWgsPerCu : kStreamWgsPerCu;
  const int lds_fit = static_cast<int>(kLdsMax / (lds > 0 ? lds : 1));
  if (lds_fit < per_cu) per_cu = lds_fit > 0 ? lds_fit : 1;
  // Persistent: as many workgroups as stay resident (a tile-count-balanced
  // grid with fewer waves, or one with more than fit, both measured slower
  // on the LM head than this one-round-uneven split).
  const int G = K / kGroup;
  const int want = (ntiles + WV - 1) / WV;
  const int cap = cu_count() * per_cu;
  const int grid = want < cap ? want : cap;
  // Waves with at most one tile compute their offset chains inline and
  // skip the workgroup's offset table and its barrier (3584x1024 M=1:
  // 4.30 -> 4.10 us); waves that stream many tiles share the table (inline
  // chains cost the LM head 0.9 us at M = 1 and 3.6 us at M = 8).
  const bool ioff = ntiles <= grid * WV;
  if (P.count == 1) {
    auto kern =
        ioff ? (G % 4 == 0 ? w4a16_stream_piece_one_kernel<PACKED, NR, SVEC, CT, Act, 4, true, WV, true>
                           : w4a16_stream_piece_one_kernel<PACKED, NR, SVEC, CT, Act, 4, false, WV, true>)
             : (G % 4 == 0 ? w4a16_stream_piece_one_kernel<PACKED, NR, SVEC, CT, Act, 4, true, WV, false>
                           : w4a16_stream_piece_one_kernel<PACKED, NR, SVEC, CT, Act, 4, false, WV, false>);
    if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(WV * 64), lds, stream, P.w[0], P.s[0], P.y[0], P.n[0],
                       ntiles, X, K, M, grid, ntiles);
    return launch_status();
  }
  auto kern =
      ioff ? (G % 4 == 0 ? w4a16_stream_piece_kernel<PACKED, NR, SVEC, CT, Act, 4, true, WV, true>
                         : w4a16_stream_piece_kernel<PACKED, NR, SVEC, CT, Act, 4, false, WV, true>)
           : (G % 4 == 0 ? w4a16_stream_piece_kernel<PACKED, NR, SVEC, CT, Act, 4, true, WV, false>
                         : w4a16_stream_piece_kernel<PACKED, NR, SVEC, CT, Act, 4, false, WV, false>);
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(WV * 64), lds, stream, P, X, K, M, grid, ntiles);
  return launch_status();
}

// Piece split plan: HG groups per piece, WV waves per workgroup; hg = 0
// when the unit split or the stream kernel serves the launch. Measured in
// graph replay over 64 distinct weight sets (us, M = 1 / 8 / 32; the stream
// or unit split kernel first): 3584x1024 4.08/4.64/7.73 -> 3.56/4.03/5.75
// with one group per wave on 8 waves; 6144x1024 4.16/4.68/7.76 -> 3.88/
// 4.28/6.67 with pieces of 2; 1024x2048 4.39/5.36/10.22 -> 4.06/4.87/8.27;
// 1024x3584 M = 8 6.49 -> 6.00. Eight waves per tile win while the tiles
// fit one per CU; beyond that pieces of 2 (four waves per tile) win up to
// the tile counts below, and the persistent stream kernel wins past them.
// 1024x3584 at M = 1 keeps the unit split (4.52 vs 4.59 us).
//
// dx: each wave loads its pieces' activation fragments straight from global
// memory into registers, so neither the LDS staging nor its barrier sits in
// front of the first MFMA (us, M = 1 / 8 / 32, LDS staging -> direct):
// 512x1024 2.94/3.56/5.35 -> 2.49/3.02/4.57; 3584x1024 3.53/4.03/5.75 ->
// 3.05/3.53/5.00; 1024x2048 4.07/4.88/8.31 -> 3.68/4.48/7.29; 6144x1024
// 3.88/4.27 -> 3.52/4.15. Sixteen-wave workgroups of four tiles at M > 16
// load x four times per CU instead of staging it once: 6144x1024 M = 32
// 6.68 -> 10.73, so they keep the staging. With direct x, one tile per
// 4-wave workgroup in pieces of 2 serves 2 <= M <= 16 past one tile per
// CU: 6144x1024 M = 8 4.28 -> 4.12, 8208x1024 4.86 (stream) -> 4.41,
// 12288x1024 4.97 (stream) -> 4.87; 16384x1024 stays on the stream kernel.
struct SplitPlan {
  int hg, wv;
  bool dx;
};


size_t split_piece_lds_bytes(int K, int M, SplitPlan p, int NP = 1) {
  const int CT = M > 16 ? 2 : 1;
  const int PPU = kUnit / p.hg;
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  const int ST = NP * U * PPU;
  const int tpr = ST >= p.wv ? 1 : p.wv / ST;
  // the file-layout staging rows at one column tile are counted for both
  // layouts (pieces of 2 or 4 groups)
  const size_t stage = M <= 16 && (p.hg == 2 || p.hg == 4)
                           ? static_cast<size_t>(p.wv) * kTileRows * (p.hg * 64 + 16)
                           : 0;
  return (p.dx ? 0 : static_cast<size_t>(M) * x_pitch(K) * 16) +
         static_cast<size_t>(tpr) * NP * U * CT * 64 * 16 * (1 + (PPU - 1) * p.hg) +
         static_cast<size_t>(tpr) * NP * U * (PPU - 1) * p.hg * 16 * 4 + stage;
}

SplitPlan split_piece_plan(int ntiles, int K, int M) {
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  const int cus = cu_count();
  SplitPlan p = {0, 0, false};
  if (M > 32) return p;
  if (ntiles <= cus && (U == 1 || U == 2 || (U == 4 && M > 1)))
    p = {U, 8, true};
  else if (U == 1 && ntiles <= (M <= 16 ? (M == 1 ? 4 : 3) * cus : 4 * cus))
    p = {2, M <= 16 ? 4 : 16, M <= 16};
  if (p.hg != 0 && split_piece_lds_bytes(K, M, p) > kLdsMax) p = {0, 0, false};
  return p;
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act, int HG, int WV, bool DX, class PT>
int launch_split_piece_t(const PT& P, const uint16_t* X, int K, int M, hipStream_t stream) {
  constexpr int PPU = kUnit / HG;
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  const int SP = U * PPU;
  const int tpr = SP >= WV ? 1 : WV / SP;
  const size_t lds = split_piece_lds_bytes(K, M, SplitPlan{HG, WV, DX});
  const int grid = (P.ntiles + tpr - 1) / tpr;
  if constexpr (std::is_same<PT, ProjOne>::value) {
    auto kern = w4a16_split_piece_one_kernel<PACKED, NR, SVEC, CT, Act, HG, WV, DX>;
    if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(WV * 64), lds, stream, P.w[0], P.s[0], P.y[0],
                       P.n[0], P.ntiles, X, K, M);
    return launch_status();
  }
  if constexpr (std::is_same<PT, ProjFour>::value) {
    auto kern = w4a16_split_piece_four_kernel<PACKED, NR, SVEC, CT, Act, HG, WV, DX>;
    if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(WV * 64), lds, stream, P.w[0], P.w[1], P.w[2],
                       P.w[3], P.tile_end[0], P.tile_end[1], P.tile_end[2], P.count, X, K, M,
                       P.s[0], P.s[1], P.s[2], P.s[3], P.y[0], P.y[1], P.y[2], P.y[3], P.n[0],
                       P.n[1], P.n[2], P.n[3], P.ntiles);
    return launch_status();
  }
  auto kern = w4a16_split_piece_kernel<PACKED, NR, SVEC, CT, Act, HG, WV, 1, DX, PT>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(WV * 64), lds, stream, P, X, K, M, M);
  return launch_status();
}

// The plans split_piece_plan can return for this accumulator shape.
template <bool PACKED, int NR, bool SVEC, int CT, class Act, class PT>
int launch_split_piece(const PT& P, const uint16_t* X, int K, int M, SplitPlan p,
                       hipStream_t stream) {
  if (p.hg == 1 && p.wv == 8 && p.dx)
    return launch_split_piece_t<PACKED, NR, SVEC, CT, Act, 1, 8, true, PT>(P, X, K, M, stream);
  if (p.hg == 2 && p.wv == 8 && p.dx)
    return launch_split_piece_t<PACKED, NR, SVEC, CT, Act, 2, 8, true, PT>(P, X, K, M, stream);
  if constexpr (CT == 1) {
    if (p.hg == 2 && p.wv == 4 && p.dx)
      return launch_split_piece_t<PACKED, NR, SVEC, CT, Act, 2, 4, true, PT>(P, X, K, M, stream);
  }
  if constexpr (NR == 4) {
    if (p.hg == 4 && p.wv == 8 && p.dx)
      return launch_split_piece_t<PACKED, NR, SVEC, CT, Act, 4, 8, true, PT>(P, X, K, M, stream);
  }
  if constexpr (CT == 2) {
    if (p.hg == 2 && p.wv == 16 && !p.dx)
      return launch_split_piece_t<PACKED, NR, SVEC, CT, Act, 2, 16, false, PT>(P, X, K, M, stream);
  }
  return CUDALM_W4A16_EVARIANT;
}

template <bool PACKED, int NR, bool SVEC, int CT, class Act = ActBf16>
int launch_split_t(const ProjTable& P, const uint16_t* X, int K, int M, hipStream_t stream) {
  const SplitPlan plan = split_piece_plan(P.ntiles, K, M);
  if (plan.hg != 0) {
    if (P.count == 1) {
      const ProjOne one = shrink_table<1>(P);
      return launch_split_piece<PACKED, NR, SVEC, CT, Act>(one, X, K, M, plan, stream);
    }
    if constexpr (std::is_same<Act, ActBf16>::value) {
      // the fused projection groups (qkv/z/b/a, q/k/v, gate/up) have <= 4
      if (P.count <= 4) {
        const ProjFour four = shrink_table<4>(P);
        return launch_split_piece<PACKED, NR, SVEC, CT, Act>(four, X, K, M, plan, stream);
      }
    }
    return launch_split_piece<PACKED, NR, SVEC, CT, Act>(P, X, K, M, plan, stream);
  }
  const size_t lds = split_kernel_lds(K, M, PACKED);
  const int ntiles = P.ntiles;
  const int tpr = split_tiles_per_round(K);
  const int grid = (ntiles + tpr - 1) / tpr;
  if (P.count == 1) {
    auto kern = w4a16_split_one_kernel<PACKED, NR, SVEC, CT, Act>;
    if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kStreamWaves * 64), lds, stream, P.w[0], P.s[0],
                       P.y[0], P.n[0], P.ntiles, X, K, M);
    return launch_status();
  }
  auto kern = w4a16_split_kernel<PACKED, NR, SVEC, CT, Act>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kStreamWaves * 64), lds, stream, P, X, K, M);
  return launch_status();
}

size_t swiglu_lds_bytes(int K, int mrows) {
  const int CT = mrows > 16 ? 2 : 1;
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  const int tpr = 2 * U >= kStreamWaves ? 1 : kStreamWaves / (2 * U);
  return stream_lds_bytes(K, mrows) + static_cast<size_t>(tpr) * 2 * U * CT * 64 * 16;
}

template <bool PACKED, int NR, bool SVEC, int CT>
int launch_swiglu_t(const ProjTable& P, const uint16_t* X, int K, int M, int mc,
                    hipStream_t stream) {
  const size_t lds = swiglu_lds_bytes(K, mc);
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  const int tpr = 2 * U >= kStreamWaves ? 1 : kStreamWaves / (2 * U);
  const int gx = (P.tile_end[0] + tpr - 1) / tpr;
  const int gy = (M + mc - 1) / mc;
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  auto kern = w4a16_swiglu_kernel<PACKED, NR, SVEC, CT>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(kStreamWaves * 64), lds, stream, P, X, K, M, mc);
  return launch_status();
}

// Activation rows per chunk of the fused kernel: up to 32 when M > 16, as
// many as the LDS holds; 0 if not even one row fits.
int swiglu_rows_per_chunk(int K, int M) {
  int mc = M > 16 ? 32 : M;
  while (mc > 0 && swiglu_lds_bytes(K, mc) > kLdsMax) --mc;
  return mc;
}

// SwiGLU through the piece split kernel (NP = 2): hg = 0 keeps the unit
// kernel above. Measured in graph replay over 32 distinct gate/up pairs
// (us, M = 1 / 8 / 32, unit kernel first): 3584x1024 5.11/5.89/9.58 ->
// 4.82 (pieces of 4 on 4 waves) / 5.80 (same) / 8.03 (pieces of 2 on 8
// waves); 9000x1024 6.77/7.67 -> 6.26/7.44, M = 32 unit kernel (12.6 vs
// 16.1); 1024x2048 M = 1/8 unit kernel (4.86 vs 5.46), M = 32 12.21 ->
// 10.53 (pieces of 2 on 16 waves).
//
// Direct activation loads (dx) pay at M <= 16 while the row tiles fit one
// per CU, best with pieces of 2 on 8 waves: 3584x1024 M = 1/8 4.82/5.81 ->
// 4.14/5.33 us, 4096x1024 M = 1 4.40 (pieces of 4, dx) -> 4.12; at M = 32
// (8.0 -> 8.6) and past one row tile per CU (9000x1024 M = 8 7.41 -> 7.83)
// the LDS staging wins.
SplitPlan swiglu_piece_plan(int nt, int K, int M) {
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  const int cus = cu_count();
  if (U == 1 && M <= 16 && nt <= cus) return {2, 8, true};
  if (U == 1 && M <= 16 && nt <= 4 * cus) return {4, 4, false};
  if (U == 1 && nt <= cus) return {2, 8, false};
  if (U == 2 && M > 16 && nt <= cus) return {2, 16, false};
  return {0, 0, false};
}

template <bool PACKED, int NR, bool SVEC, int CT, int HG, int WV, bool DX>
int launch_swiglu_piece_t(const ProjTable& P, const uint16_t* X, int K, int M, int mc,
                          hipStream_t stream) {
  constexpr int PPU = kUnit / HG;
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  const int ST = 2 * U * PPU;
  const int tpr = ST >= WV ? 1 : WV / ST;
  const size_t lds = split_piece_lds_bytes(K, mc, SplitPlan{HG, WV, DX}, 2);
  const int gx = (P.tile_end[0] + tpr - 1) / tpr;
  const int gy = (M + mc - 1) / mc;
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  auto kern = w4a16_split_piece_pair_kernel<PACKED, NR, SVEC, CT, HG, WV, DX>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(WV * 64), lds, stream, P.w[0], P.w[1], P.tile_end[0],
                     P.count, X, K, M, mc, P.s[0], P.s[1], P.y[0], P.y[1], P.n[0], P.n[1],
                     P.ntiles);
  return launch_status();
}

template <bool PACKED>
int launch_swiglu(const ProjTable& P, const uint16_t* X, int K, int M, hipStream_t stream) {
  const int G = K / kGroup;
  const bool svec = !PACKED && G % 8 == 0 && aligned(P.s[0], 16) && aligned(P.s[1], 16);
  const SplitPlan plan = swiglu_piece_plan(P.tile_end[0], K, M);
  if (plan.hg != 0) {
    int mc = M > 16 ? 32 : M;
    while (mc > 0 && split_piece_lds_bytes(K, mc, plan, 2) > kLdsMax) --mc;
    // a plan for M > 16 needs 32-row chunks (CT = 2)
    if (mc > 0 && (M <= 16 || mc > 16)) {
#define W4A16_SWP(NR, CT, HG, WV, DX)                                                      \
  (svec ? launch_swiglu_piece_t<PACKED, NR, true, CT, HG, WV, DX>(P, X, K, M, mc, stream) \
        : launch_swiglu_piece_t<PACKED, NR, false, CT, HG, WV, DX>(P, X, K, M, mc, stream))
      if (mc > 16)
        return plan.wv == 16 ? W4A16_SWP(4, 2, 2, 16, false) : W4A16_SWP(4, 2, 2, 8, false);
      if (M == 1) return plan.dx ? W4A16_SWP(1, 1, 2, 8, true) : W4A16_SWP(1, 1, 4, 4, false);
      return plan.dx ? W4A16_SWP(4, 1, 2, 8, true) : W4A16_SWP(4, 1, 4, 4, false);
#undef W4A16_SWP
    }
  }
  const int mc = swiglu_rows_per_chunk(K, M);
  if (mc < 1) return CUDALM_W4A16_ERANGE;
#define W4A16_SWIGLU(NR, CT)                                                       \
  (svec ? launch_swiglu_t<PACKED, NR, true, CT>(P, X, K, M, mc, stream)           \
        : launch_swiglu_t<PACKED, NR, false, CT>(P, X, K, M, mc, stream))
  if (mc > 16) return W4A16_SWIGLU(4, 2);
  if (M == 1) return W4A16_SWIGLU(1, 1);
  return W4A16_SWIGLU(4, 1);
#undef W4A16_SWIGLU
}

// Unit-parallel (split) when the tiles alone leave most of the machine
// idle and each tile has several units; otherwise tile-serial streaming.
bool prefer_split(const ProjTable& P, int K, int M, bool packed) {
  const int U = (K / kGroup + kUnit - 1) / kUnit;
  return split_piece_plan(P.ntiles, K, M).hg != 0 ||
         (U >= 2 && split_fits(K, M, packed) && P.ntiles < 2 * cu_count());
}

template <bool PACKED, bool SPLIT, class Act = ActBf16>
int launch_stream_any(const ProjTable& P, const uint16_t* X, int K, int M, hipStream_t stream) {
  const int G = K / kGroup;
  bool svec = false;
  if (!PACKED && G % 8 == 0) {
    svec = true;
    for (int j = 0; j < P.count; ++j) svec = svec && aligned(P.s[j], 16);
  }
#define W4A16_LAUNCH(NR, SV, CT)                                          \
  (SPLIT ? launch_split_t<PACKED, NR, SV, CT, Act>(P, X, K, M, stream)    \
         : launch_stream_t<PACKED, NR, SV, CT, Act>(P, X, K, M, stream))
  if (M > 16) return svec ? W4A16_LAUNCH(4, true, 2) : W4A16_LAUNCH(4, false, 2);
  if (M == 1) return svec ? W4A16_LAUNCH(1, true, 1) : W4A16_LAUNCH(1, false, 1);
  return svec ? W4A16_LAUNCH(4, true, 1) : W4A16_LAUNCH(4, false, 1);
#undef W4A16_LAUNCH
}

template <bool PACKED, class Act = ActBf16>
int launch_stream(const ProjTable& P, const uint16_t* X, int K, int M, hipStream_t stream) {
  return prefer_split(P, K, M, PACKED) ? launch_stream_any<PACKED, true, Act>(P, X, K, M, stream)
                               : launch_stream_any<PACKED, false, Act>(P, X, K, M, stream);
}

ProjTable single_table(const uint8_t* W, const uint16_t* S, uint16_t* Y, int N) {
  ProjTable P = {};
  P.w[0] = W;
  P.s[0] = S;
  P.y[0] = Y;
  P.n[0] = N;
  P.tile_end[0] = (N + kTileRows - 1) / kTileRows;
  P.count = 1;
  P.ntiles = P.tile_end[0];
  return P;
}

template <int RB, int CT, int WN, int WM, int GPC, bool PACKED>
int launch_tile(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N, int K,
                int M, hipStream_t stream) {
  constexpr int CM = WM * CT * 16;
  constexpr int KC = GPC * kGroup;
  const int mrows = M < CM ? M : CM;
  const size_t lds = static_cast<size_t>(mrows) * x_pitch(KC) * 16;
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int gx = (ntiles + WN * RB - 1) / (WN * RB);
  const int gy = (M + CM - 1) / CM;
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  auto kern = w4a16_tile_kernel<RB, CT, WN, WM, GPC, PACKED>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(WN * WM * 64), lds, stream, W, S, X, Y, N, K, M);
  return launch_status();
}

template <int RB, int CT, int WV, bool PACKED, int KS = 1, bool IOFF = false>
int launch_gemm_unit(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                     int K, int M, hipStream_t stream) {
  constexpr int TM = CT * 16;
  const size_t xbytes = static_cast<size_t>(TM) * x_pitch(kUnit * kGroup) * 16;
  const size_t lds = KS * (xbytes + static_cast<size_t>(kUnit) * CT * 16 * sizeof(float));
  const int G = K / kGroup;
  if constexpr (KS > 1) {
    // every slice keeps at most kSliceMaxUnits partials, and all of them
    // must fit the x buffers they are parked in
    const int U = (G + kUnit - 1) / kUnit;
    if (U > KS * kSliceMaxUnits ||
        static_cast<size_t>(U) * WV * RB * CT * 64 * 16 > KS * xbytes)
      return launch_gemm_unit<RB, CT, WV, PACKED, 1, IOFF>(W, S, X, Y, N, K, M, stream);
  }
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const int gx = (ntiles + WV * RB - 1) / (WV * RB);
  const int gy = (M + TM - 1) / TM;
  if (gy > 65535) return CUDALM_W4A16_ERANGE;
  const bool svec = !PACKED && G % 8 == 0 && aligned(S, 16);
  auto kern = svec ? w4a16_gemm_unit_kernel<RB, CT, WV, PACKED, true, KS, IOFF>
                   : w4a16_gemm_unit_kernel<RB, CT, WV, PACKED, false, KS, IOFF>;
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(WV * KS * 64), lds, stream, W, S, X, Y, N, K, M);
  return launch_status();
}

// Prefill chunks (M >= 33). The 32 x 32 MFMA GEMM (w4a16_gemm.hip: 32
// activation rows x 256 weight rows per 8-wave workgroup) serves K <= 1024
// when its workgroups fill between 3/4 and all of the CUs in one round
// (3584x1024 and 4096x1024 at M = 512: 10.3 -> 9.6-9.9 us, 10.7 -> 9.5-10.0 us);
// elsewhere the 16 x 16 unit GEMM is faster (one round of 32 x 256 tiles
// leaves too many CUs idle below that, and past one round it takes two).
// Unit GEMM tiles: 128 x 32 of 8 waves while they fill most of the CUs,
// else 64 x 32 of 4 waves, with two k-slices of 4 waves when K spans
// several units (1024x3584 at M = 512: 16.7 -> 14.6 us). The 4-wave tiles
// run their offset chains inline (512x1024x512 5.8 -> 5.5 us, 1024x3584x512
// 14.4 -> 13.8 us); inline chains cost the 8-wave tiles 0.6 us at
// 3584x1024x512, so those keep the table.
template <bool PACKED>
int launch_prefill(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N, int K,
                   int M, hipStream_t stream) {
  const int cus = cu_count();
  if (K == kUnit * kGroup && prefill_split_waves(N, M, cus, PACKED) != 0)
    return launch_prefill32<PACKED>(W, S, X, Y, N, K, M, stream);
  if (K < kUnit * kGroup) {
    const long long wgs32 = static_cast<long long>((N + 255) / 256) * ((M + 31) / 32);
    if (4 * wgs32 >= 3LL * cus && wgs32 <= cus)
      return launch_prefill32<PACKED>(W, S, X, Y, N, K, M, stream);
  }
  const long long wgs = static_cast<long long>((N + 127) / 128) * ((M + 31) / 32);
  // (crossover measured between 128 and 168 workgroups of 128 x 32:
  // 2048x1024x256 5.7 vs 6.9 us, 3584x1024x192 7.4 vs 6.9 us)
  if (5 * wgs >= 3LL * cus) return launch_gemm_unit<1, 2, 8, PACKED>(W, S, X, Y, N, K, M, stream);
  if (K > kUnit * kGroup)
    return launch_gemm_unit<1, 2, 4, PACKED, 2, true>(W, S, X, Y, N, K, M, stream);
  return launch_gemm_unit<1, 2, 4, PACKED, 1, true>(W, S, X, Y, N, K, M, stream);
}

template <class Act = ActBf16>
int launch_bytewise(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                    int K, int M, hipStream_t stream) {
  if (M > 65535) return CUDALM_W4A16_ERANGE;
  hipLaunchKernelGGL(w4a16_bytewise_kernel<Act>, dim3((N + 3) / 4, M), dim3(256), 0, stream, W,
                     reinterpret_cast<const uint8_t*>(S), reinterpret_cast<const uint8_t*>(X),
                     reinterpret_cast<uint8_t*>(Y), N, K);
  return launch_status();
}


// The piece split with activations in registers needs no LDS for x, so it
// also serves 17 <= M <= 32 when x does not fit the LDS (1024x3584 at
// M = 32: one launch instead of two 16-row passes).
bool piece_direct(int ntiles, int K, int M) {
  const SplitPlan p = split_piece_plan(ntiles, K, M);
  return p.hg != 0 && p.dx;
}

template <bool PACKED>
int dispatch(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N, int K,
             int M, int variant, hipStream_t stream) {
  if (variant == CUDALM_W4A16_VARIANT_AUTO) {
    if (stream_fits(K, M, PACKED) || piece_direct((N + kTileRows - 1) / kTileRows, K, M)) {
      const ProjTable P = single_table(W, S, Y, N);
      return launch_stream<PACKED>(P, X, K, M, stream);
    } else if (M <= 32 && M > 16) {
      // x does not fit in LDS at once: 16-row column passes
      for (int m0 = 0; m0 < M; m0 += 16) {
        const int mc = M - m0 < 16 ? M - m0 : 16;
        if (int rc = dispatch<PACKED>(W, S, X + static_cast<size_t>(m0) * K,
                                      Y + static_cast<size_t>(m0) * N, N, K, mc,
                                      CUDALM_W4A16_VARIANT_AUTO, stream))
          return rc;
      }
      return CUDALM_W4A16_OK;
    } else if (M <= 16) {
      variant = CUDALM_W4A16_VARIANT_TILE16;
    } else {
      variant = CUDALM_W4A16_VARIANT_PREFILL;
    }
  }
  switch (variant) {
    case CUDALM_W4A16_VARIANT_STREAM:
      if (!stream_fits(K, M, PACKED)) return CUDALM_W4A16_EVARIANT;
      return launch_stream_any<PACKED, false>(single_table(W, S, Y, N), X, K, M, stream);
    case CUDALM_W4A16_VARIANT_SPLIT:
      if (!split_fits(K, M, PACKED) && split_piece_plan((N + kTileRows - 1) / kTileRows, K, M).hg == 0)
        return CUDALM_W4A16_EVARIANT;
      return launch_stream_any<PACKED, true>(single_table(W, S, Y, N), X, K, M, stream);
    case CUDALM_W4A16_VARIANT_TILE16:
      return launch_tile<1, 1, 4, 1, 8, PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_TILE32:
      return launch_tile<1, 2, 4, 1, 8, PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_PREFILL:
      return launch_prefill<PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_PREFILL32:
      return launch_prefill32<PACKED>(W, S, X, Y, N, K, M, stream);
    case CUDALM_W4A16_VARIANT_BYTEWISE:
      if (PACKED) return CUDALM_W4A16_EVARIANT;
      return launch_bytewise(W, S, X, Y, N, K, M, stream);
    default:
      return CUDALM_W4A16_EVARIANT;
  }
}

// fp16-activation twin: M rows in chunks that fit the stream kernels' LDS
// (one launch when M <= 32 and x fits), the byte-wise kernel for
// misaligned file-layout bases.
template <bool PACKED>
int f16_dispatch(const uint8_t* W, const uint16_t* S, const uint16_t* X, uint16_t* Y, int N,
                 int K, int M, bool vec_ok, hipStream_t stream) {
  if (!vec_ok) return launch_bytewise<ActF16>(W, S, X, Y, N, K, M, stream);
  int mc = M < 32 ? M : 32;
  while (mc > 0 && !stream_fits(K, mc, PACKED)) --mc;
  if (mc < 1) return CUDALM_W4A16_ERANGE;
  for (int m0 = 0; m0 < M; m0 += mc) {
    const int rows = M - m0 < mc ? M - m0 : mc;
    const ProjTable P = single_table(W, S, Y + static_cast<size_t>(m0) * N, N);
    if (int rc = launch_stream<PACKED, ActF16>(P, X + static_cast<size_t>(m0) * K, K, rows, stream))
      return rc;
  }
  return CUDALM_W4A16_OK;
}

}  // namespace


extern "C" {

int cudalm_w4a16_version(void) { return 300; }

const char* cudalm_w4a16_strerror(int code) {
  switch (code) {
    case CUDALM_W4A16_OK: return "ok";
    case CUDALM_W4A16_EINVAL:
      return "invalid shape: requires N >= 1, M >= 1, K > 0 (W4A16 entry points: K % 128 == 0)";
    case CUDALM_W4A16_ENULL: return "null pointer argument";
    case CUDALM_W4A16_EALIGN:
      return "base misaligned (prepacked W4A16 buffers: 16 bytes; bf16 buffers: 2 bytes)";
    case CUDALM_W4A16_ELAUNCH: return "HIP kernel launch failed";
    case CUDALM_W4A16_ERANGE: return "shape exceeds the kernels' index range";
    case CUDALM_W4A16_EVARIANT: return "unknown or inapplicable kernel variant";
    case -7: return "weight file breaks a .cudalm v2 container rule";
    case -8: return "weight file could not be opened or mapped";
    case -9: return "tensor not found, or not of the expected dtype / shape";
    case CUDALM_W4A16_ETIMEOUT: return "a chain stage waited past its bound (outputs unspecified)";
    default: return "unknown error code";
  }
}

int cudalm_w4a16_gemv_bf16_variant(const uint8_t* weight, const uint16_t* scale, const uint16_t* x,
                                   uint16_t* y, int N, int K, int M, int variant,
                                   hipStream_t stream) {
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
  return static_cast<size_t>((N + 15) / 16) * packed_tile_bytes(K / kGroup);
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

int cudalm_w4a16_gemv_bf16_multi(const cudalm_w4a16_proj* projs, int count, const uint16_t* x,
                                 int K, int M, int prepacked, hipStream_t stream) {
  if (count < 1 || count > CUDALM_W4A16_MAX_PROJ) return CUDALM_W4A16_EINVAL;
  if (!projs || !x) return CUDALM_W4A16_ENULL;
  bool vec_ok = aligned(x, 16);
  for (int j = 0; j < count; ++j) {
    if (int rc = check_shape(projs[j].N, K, M)) return rc;
    if (!projs[j].weight || !projs[j].y || (!prepacked && !projs[j].scale)) return CUDALM_W4A16_ENULL;
    vec_ok = vec_ok && aligned(projs[j].weight, 16) && aligned(projs[j].y, 2) &&
             (prepacked || aligned(projs[j].scale, 2));
  }
  if (prepacked && !vec_ok) return CUDALM_W4A16_EALIGN;
  long long tiles = 0;
  for (int j = 0; j < count; ++j) tiles += (projs[j].N + kTileRows - 1) / kTileRows;
  if (!vec_ok || tiles > (1LL << 30) ||
      (!stream_fits(K, M, prepacked) && !piece_direct(static_cast<int>(tiles), K, M))) {
    // not one fused launch: one call per projection (same bits)
    for (int j = 0; j < count; ++j) {
      const int rc =
          prepacked ? cudalm_w4a16_gemv_bf16_prepacked(projs[j].weight, x, projs[j].y, projs[j].N,
                                                       K, M, stream)
                    : cudalm_w4a16_gemv_bf16(static_cast<const uint8_t*>(projs[j].weight),
                                             projs[j].scale, x, projs[j].y, projs[j].N, K, M,
                                             stream);
      if (rc) return rc;
    }
    return CUDALM_W4A16_OK;
  }
  ProjTable P = {};
  int acc_tiles = 0;
  for (int j = 0; j < count; ++j) {
    P.w[j] = static_cast<const uint8_t*>(projs[j].weight);
    P.s[j] = projs[j].scale;
    P.y[j] = projs[j].y;
    P.n[j] = projs[j].N;
    acc_tiles += (projs[j].N + kTileRows - 1) / kTileRows;
    P.tile_end[j] = acc_tiles;
  }
  P.count = count;
  P.ntiles = acc_tiles;
  return prepacked ? launch_stream<true>(P, x, K, M, stream) : launch_stream<false>(P, x, K, M, stream);
}

int cudalm_w4a16_gemv_f16(const uint8_t* weight, const uint16_t* scale, const uint16_t* x,
                          uint16_t* y, int N, int K, int M, hipStream_t stream) {
  if (int rc = check_shape(N, K, M)) return rc;
  if (!weight || !scale || !x || !y) return CUDALM_W4A16_ENULL;
  const bool vec_ok = aligned(weight, 16) && aligned(x, 16) && aligned(scale, 2) && aligned(y, 2);
  return f16_dispatch<false>(weight, scale, x, y, N, K, M, vec_ok, stream);
}

int cudalm_w4a16_gemv_f16_prepacked(const void* packed, const uint16_t* x, uint16_t* y, int N,
                                    int K, int M, hipStream_t stream) {
  if (int rc = check_shape(N, K, M)) return rc;
  if (!packed || !x || !y) return CUDALM_W4A16_ENULL;
  if (!aligned(packed, 16) || !aligned(x, 16) || !aligned(y, 2)) return CUDALM_W4A16_EALIGN;
  return f16_dispatch<true>(static_cast<const uint8_t*>(packed), nullptr, x, y, N, K, M, true,
                            stream);
}

int cudalm_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* y, size_t n,
                         hipStream_t stream) {
  if (n == 0) return CUDALM_W4A16_OK;
  if (!gate || !up || !y) return CUDALM_W4A16_ENULL;
  if (!aligned(gate, 2) || !aligned(up, 2) || !aligned(y, 2)) return CUDALM_W4A16_EALIGN;
  const size_t threads = (n + 7) / 8;
  const size_t blocks = (threads + 255) / 256;
  if (blocks > 0x7FFFFFFFu) return CUDALM_W4A16_ERANGE;
  const int vec = aligned(gate, 16) && aligned(up, 16) && aligned(y, 16);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     gate, up, y, n, vec);
  return launch_status();
}

int cudalm_w4a16_swiglu_bf16(const void* gate_weight, const uint16_t* gate_scale,
                             const void* up_weight, const uint16_t* up_scale, const uint16_t* x,
                             uint16_t* y, int N, int K, int M, int prepacked,
                             hipStream_t stream) {
  if (int rc = check_shape(N, K, M)) return rc;
  if (!gate_weight || !up_weight || !x || !y || (!prepacked && (!gate_scale || !up_scale)))
    return CUDALM_W4A16_ENULL;
  if (static_cast<long long>((N + kTileRows - 1) / kTileRows) * 2 > (1LL << 30))
    return CUDALM_W4A16_ERANGE;
  const bool vec_ok = aligned(gate_weight, 16) && aligned(up_weight, 16) && aligned(x, 16) &&
                      aligned(y, 2) &&
                      (prepacked || (aligned(gate_scale, 2) && aligned(up_scale, 2)));
  if (!vec_ok) return CUDALM_W4A16_EALIGN;
  ProjTable P = {};
  const int nt = (N + kTileRows - 1) / kTileRows;
  P.w[0] = static_cast<const uint8_t*>(gate_weight);
  P.s[0] = gate_scale;
  P.w[1] = static_cast<const uint8_t*>(up_weight);
  P.s[1] = up_scale;
  P.y[0] = P.y[1] = y;
  P.n[0] = P.n[1] = N;
  P.tile_end[0] = nt;
  P.tile_end[1] = 2 * nt;
  P.count = 2;
  P.ntiles = 2 * nt;
  return prepacked ? launch_swiglu<true>(P, x, K, M, stream)
                   : launch_swiglu<false>(P, x, K, M, stream);
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
    case CUDALM_W4A16_VARIANT_STREAM:
      return regs_of(w4a16_stream_piece_one_kernel<true, 1, false, 1, ActBf16, 4, true, 4, false>);
    case CUDALM_W4A16_VARIANT_TILE16: return regs_of(w4a16_tile_kernel<1, 1, 4, 1, 8, true>);
    case CUDALM_W4A16_VARIANT_TILE32: return regs_of(w4a16_tile_kernel<1, 2, 4, 1, 8, true>);
    case CUDALM_W4A16_VARIANT_PREFILL: return regs_of(w4a16_gemm_unit_kernel<1, 2, 8, true, false>);
    case CUDALM_W4A16_VARIANT_PREFILL32: return prefill32_regs();
    case CUDALM_W4A16_VARIANT_BYTEWISE: return regs_of(w4a16_bytewise_kernel<ActBf16>);
    case CUDALM_W4A16_VARIANT_SPLIT: return regs_of(w4a16_split_kernel<true, 1, false, 1>);
    case CUDALM_W4A16_VARIANT_SWIGLU: return regs_of(w4a16_swiglu_kernel<true, 1, false, 1>);
    default: return -1;
  }
}

}  // extern "C"
