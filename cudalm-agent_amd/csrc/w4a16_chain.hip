// Stage chains: an ordered list of W4A16 projection stages run by one
// persistent launch (gfx950). Declared in include/cudalm_w4a16.h
// (cudalm_w4a16_chain_*).
//
// Why: a decode step runs ~100 dependent projection launches
// (src/runtime/qwen35_model.cpp:469-491, qwen35_deltanet.cpp:166-251).
// Every launch pays a fixed cost: dispatch and completion between graph
// nodes, the kernel-argument reads, the cold weight stream. In a chain the
// workgroups stay resident; each stage's weight fragments are loaded into
// registers before the stage waits for its dependency, so a stage's
// critical path is the hand-off (flag seen -> x loaded -> MFMA -> outputs
// stored -> flag written), not a launch.
//
// Arithmetic: per output the same operation sequence as every other
// kernel of the library (w4a16_kernels.hip): per group the offset chain
// (-1.5 * sum x, four MFMAs against a constant operand) seeds the
// four-step weight chain of the exact 1.5 + q/16 decode; within an 8-group
// unit part = fma(s_g, tmp_g, part) from 0 in group order; the unit
// partials are summed from 0 in unit order; y = bf16_rne(16 * total). So a
// chain stage writes the bits of cudalm_w4a16_gemv_bf16 on its inputs.
//
// Work split: a stage's 16-row tiles go to `nwg` consecutive workgroups
// (rotating through the grid from stage to stage, so a workgroup idle in
// the current stage is already fetching its next stage's weights), up to
// `tpw` tiles per workgroup and round. Wave w of a workgroup owns groups
// w, w+8, w+16, w+24 of every one of its tiles. Before the wait it loads and
// decodes those weight fragments (at most 4: 64 VGPRs decoded) and parks the
// fp16 scales in LDS; after the wait it loads x for its groups once, builds
// their offset chains once, runs the four-step weight chain of every tile
// and parks each group result in LDS; after a barrier wave j continues tile
// j's fma chain in group order and stores the tile.
//
// Hand-off protocol (device scope, no cache-wide maintenance):
//   * outputs are stored with device-coherent stores (sc1) and each storing
//     wave waits for its stores to complete before the workgroup barrier;
//     then one lane writes the workgroup's flag, flags[stage][slot] = epoch,
//     every flag in its own 128-byte line;
//   * a waiting workgroup's first wave polls the dependency's flags with
//     device-coherent loads until every one equals the epoch, then a barrier;
//     x is then read with device-coherent loads (it may be another stage's
//     output);
//   * the epoch is this launch's number: each workgroup keeps its own epoch
//     word in the workspace, reads it at the start (+1) and stores it back
//     at its exit; every workgroup of the fixed grid runs every launch, so
//     the words advance together. No flag is ever cleared, a replay needs
//     no memset, and no atomic sits at the exit (with a device-wide
//     two-level exit counter instead, a two-stage chain took 12.7 rather
//     than 11.9 us);
//   * every wait is bounded (~0.5 s of s_memrealtime by default, settable
//     with cudalm_w4a16_chain_set_wait_bound) and gives up at once
//     when another wait has failed: it then sets the workspace error word
//     and the stage proceeds, so every wave exits; the host reads the word
//     with cudalm_w4a16_chain_status.
// Flags and epochs are written with vector stores, the error word with a
// vector atomic. The grid is the number of workgroups that are resident at
// once, so no workgroup waits on one that cannot be scheduled.
//
// Measured per stage of the M = 1 census chain (s_memrealtime probes, one
// box): last flag of stage s-1 -> stage s's wait done 1.4 us; x loaded and
// offsets 0.5 us; weight chains parked 0.4 us; reduced, stored and
// acknowledged 0.8 us; 3.3 us per stage against ~3.9 us per graph-launched
// projection group.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <type_traits>
#include <vector>

#include "cudalm_w4a16.h"
#include "hip_common.h"
#include "w4a16_device.h"

namespace {

using namespace cudalm_hip;

constexpr int kChainWaves = 8;        // waves per workgroup
constexpr int kChainProj = 4;         // projections per stage (sharing x)
// Weight fragments (one 16-byte slice of one group of one tile) a wave holds
// per round, decoded before the wait (16 VGPRs each): what the activations
// leave of the register budget (256 per lane at two waves per SIMD). Eight
// fragments spill at K = 1024; four do not.
__host__ __device__ constexpr int chain_frag(int gpw, int ct) { return (void)gpw, (void)ct, 4; }
// With four groups per wave and two column tiles the activations alone take
// 128 VGPRs: that path decodes each fragment after the wait instead.
__host__ __device__ constexpr bool chain_predecode(int gpw, int ct) { return !(gpw == 4 && ct == 2); }
constexpr int kChainGpw = 4;          // groups per wave (K <= 4096)
constexpr int kChainMaxWg = 256;      // workgroups per stage (flags polled 4 per lane)
constexpr int kChainFlagSlots = 256;  // flags per stage
constexpr int kChainFlagStride = 32;  // u32 words between flags: one 128-byte line each
constexpr int kChainMaxGrid = 2048;  // workgroups of a chain launch (at most)

// Workspace: [header 9 KB][stage table, 256 B per stage][flags, 32 KB per stage]
// header: words at byte offsets 64 (error) and 192 (wait bound), then from
// 1024 one epoch word per workgroup of the grid.
constexpr size_t kErrorOff = 64, kBoundOff = 192, kEpochsOff = 1024;
constexpr size_t kChainHeader = kEpochsOff + kChainMaxGrid * 4;
static_assert(kChainHeader % 256 == 0, "the stage table stays 256 B aligned");
constexpr uint32_t kDefaultWaitTicks = 50000000u;  // ~0.5 s of s_memrealtime (100 MHz)

struct alignas(256) ChainStage {
  const uint8_t* w[kChainProj];
  const uint16_t* s[kChainProj];
  uint16_t* y[kChainProj];
  const uint16_t* x;
  uint16_t* act;  // SwiGLU epilogue output, or null
  int n[kChainProj];
  int tile_end[kChainProj];
  int count, K, dep, ntiles;
  int first, nwg, tpw, dep_nwg;
};
static_assert(sizeof(ChainStage) == 256, "stage table stride");

__host__ __device__ inline size_t chain_table_bytes(int n) { return static_cast<size_t>(n) * sizeof(ChainStage); }
size_t chain_flag_bytes(int n) {
  return static_cast<size_t>(n) * kChainFlagSlots * kChainFlagStride * 4;
}

// ---------------------------------------------------------------------------
// device side
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t ld_dev_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes at byte offset `off` of a buffer, device-coherent (sc1).
__device__ __forceinline__ u32x4_t ld_dev_x16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           0x7FFFFFFF, 0x00020000);
}

// The projection that owns stage tile t: every field is read at a constant
// offset and picked with selects (no data-dependent scalar load chain). A
// SwiGLU stage interleaves its two projections (tile t is row tile t / 2 of
// gate for even t, of up for odd t), so a workgroup's round holds whole
// gate/up pairs.
struct StageProj {
  const uint8_t* w;
  const uint16_t* s;
  uint16_t* y;
  int n;
  int begin;  // first stage tile of the projection
};

__device__ __forceinline__ StageProj stage_proj(const ChainStage& S, int t, bool epi) {
  StageProj v = {S.w[0], S.s[0], S.y[0], S.n[0], 0};
  if (epi) {
    if (t & 1) {
      v.w = S.w[1];
      v.s = S.s[1];
    }
    v.begin = t - (t >> 1);
    return v;
  }
#pragma unroll
  for (int k = 1; k < kChainProj; ++k) {
    if (k < S.count && t >= S.tile_end[k - 1]) {
      v.w = S.w[k];
      v.s = S.s[k];
      v.y = S.y[k];
      v.n = S.n[k];
      v.begin = S.tile_end[k - 1];
    }
  }
  return v;
}

// Wave-level wait until the flags of workgroups 0..n-1 of a stage all equal
// e. Every flag has its own 128-byte line: flags that share a line are
// written one after another by the memory system (64 producers on one line
// measured 2.6 us from the last store to its detection, on separate lines
// 0.95 us). Lane l polls workgroups l, l+64, l+128, l+192 with
// device-coherent loads. Returns false on a timeout (after posting the
// error) or when another wait already failed.
__device__ bool chain_wait(const uint32_t* flags, int n, uint32_t e, uint32_t* err, uint32_t ticks) {
  const int lane = threadIdx.x & 63;
  long long deadline = 0;
  for (int it = 0;; ++it) {
    bool ok = true;
#pragma unroll
    for (int q = 0; q < kChainMaxWg / 64; ++q) {
      const int j = lane + 64 * q;
      if (j < n) ok = ok && ld_dev_u32(flags + j * kChainFlagStride) == e;
    }
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
    if ((it & 63) == 63) {
      if (ld_dev_u32(err) != 0) return false;  // another wait has failed: give up at once
      const long long now = __builtin_amdgcn_s_memrealtime();
      if (deadline == 0) {
        deadline = now + static_cast<long long>(ticks);
      } else if (now > deadline) {
        if (lane == 0) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
  }
}

// Park area of one round: tile j, group g, column tile ct at
// [(j * G + g) * CT + ct][64 lanes] (NR == 1 parks one float per lane, row 0
// being the only output row; else a f32x4), then 16 scales per (j, g), then
// the SwiGLU exchange: the bf16 up outputs of up to kChainPairs gate/up tile
// pairs, [pair][ct * NR + r][64 lanes] u32.
constexpr int kChainPairs = 2;
size_t chain_lds_bytes(int M, int gt) {
  const int NR = M == 1 ? 1 : 4, CT = M > 16 ? 2 : 1;
  return static_cast<size_t>(gt) * (static_cast<size_t>(CT) * 64 * (NR == 1 ? 4 : 16) + 64) +
         static_cast<size_t>(kChainPairs) * CT * NR * 64 * 4;
}

// One stage of the chain for one workgroup (slot = its index among the
// stage's workgroups); GPW = groups per wave, ceil(G / 8) rounded up to 1, 2
// or 4, a compile-time constant so every register array is indexed
// statically.
template <bool PACKED, int NR, int CT, int GPW>
__device__ __forceinline__ void chain_stage(const ChainStage& S, int slot, int M, int gt_max,
                                            f32x4_t* lds_park, uint32_t* flags, uint32_t e,
                                            uint32_t* err, uint32_t ticks) {
  using Park = typename std::conditional<NR == 1, float, f32x4_t>::type;
  constexpr int kChainFrag = chain_frag(GPW, CT);
  // At two column tiles the lane index is made opaque per stage: otherwise
  // the compiler hoists every lane-derived address and row mask of every
  // stage path out of the stage loop, and those spill to scratch (with one
  // column tile the hoisted values fit, and hoisting them is faster).
  int tid = static_cast<int>(threadIdx.x);
  if constexpr (CT == 2) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = wave_id();
  const int i = lane & 15, a = lane >> 4;
  const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const int K = S.K;
  const int G = K >> 7;
  const bool epi = S.act != nullptr;  // read once, before the wait
  constexpr int gpw = GPW;
  const int tpw = S.tpw;
  const int ntl = S.ntiles;
  const int U = (G + kUnit - 1) / kUnit;
  Park* tmps = reinterpret_cast<Park*>(lds_park);
  float* scs = reinterpret_cast<float*>(tmps + static_cast<size_t>(gt_max) * CT * 64);
  uint32_t* xch = reinterpret_cast<uint32_t*>(scs + static_cast<size_t>(gt_max) * 16);
  // this wave's activation fragments and offset chains, per owned group
  u32x4_t xa[GPW][CT][4];
  // The offset chains are kept for the round's tiles, except where one tile
  // per round uses each once and the registers are short (four groups per
  // wave, two column tiles): there they are built where they are used.
  constexpr bool KEEP_OFF = !(GPW == 4 && CT == 2);
  f32x4_t off[KEEP_OFF ? GPW : 1][CT];
  bool have_x = false;
  for (int c = slot; c * tpw < ntl; c += S.nwg) {
    const int t0 = c * tpw;
    const int tn = min(tpw, ntl - t0);
    // weight fragment f = j * gpw + q: tile t0 + j, group wave + 8 q
    u32x4_t wf[kChainFrag];
    uint32_t sf[kChainFrag];
#pragma unroll
    for (int f = 0; f < kChainFrag; ++f) {
      const int j = f / gpw, q = f - j * gpw;
      const int g = wave + kChainWaves * q;
      if (j < tn && g < G) {
        const int t = t0 + j;
        const StageProj v = stage_proj(S, t, epi);
        const int rt = t - v.begin;
        if constexpr (PACKED) {
          const uint8_t* tile = v.w + static_cast<size_t>(rt) * packed_tile_bytes(G);
          wf[f] = __builtin_nontemporal_load(
              reinterpret_cast<const u32x4_t*>(tile + static_cast<size_t>(g) * 1024 + lane * 16));
          sf[f] = *reinterpret_cast<const uint16_t*>(tile + static_cast<size_t>(G) * 1024 +
                                                     i * packed_scale_pitch(G) + 2 * g);
        } else {
          const int row = min(rt * kTileRows + i, v.n - 1);
          wf[f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
              v.w + static_cast<size_t>(row) * (K >> 1) + g * 64 + a * 16));
          sf[f] = v.s[static_cast<size_t>(row) * G + g];
        }
      }
    }
    // Decode the weights and park the scales while the dependency is still
    // running: what remains after x arrives is the MFMA chains.
    constexpr bool PRE = chain_predecode(GPW, CT);
    u32x4_t bw[PRE ? kChainFrag : 1][4];
#pragma unroll
    for (int f = 0; f < kChainFrag; ++f) {
      const int j = f / gpw, q = f - j * gpw;
      const int g = wave + kChainWaves * q;
      if (j < tn && g < G) {
        if constexpr (PRE)
#pragma unroll
          for (int d = 0; d < 4; ++d) bw[f][d] = decode_nibbles<PACKED>(wf[f][d]);
        if (a == 0) scs[(static_cast<size_t>(j) * G + g) * 16 + i] = half_bits_to_f32(sf[f]);
      }
    }
    if (!have_x) {
      // first round: wait for the stage x depends on, then x and the offsets
      have_x = true;
      if (S.dep >= 0) {
        if (wave == 0)
          chain_wait(flags + S.dep * kChainFlagSlots * kChainFlagStride, S.dep_nwg, e, err, ticks);
        __syncthreads();
      }
      const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(S.x);
#pragma unroll
      for (int q = 0; q < GPW; ++q) {
        const int g = wave + kChainWaves * q;
        if (q < gpw && g < G) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            const uint32_t base =
                2u * (static_cast<uint32_t>(min(ct * 16 + i, M - 1)) * static_cast<uint32_t>(K) +
                      static_cast<uint32_t>(g * kGroup + 32 * a));
#pragma unroll
            for (int d = 0; d < 4; ++d) xa[q][ct][d] = pair_order(ld_dev_x16(xr, base + 16 * d));
          }
        }
      }
      if constexpr (KEEP_OFF)
#pragma unroll
        for (int q = 0; q < GPW; ++q)
          if (q < gpw && wave + kChainWaves * q < G)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) off[q][ct] = group_offset(xa[q][ct]);
    }
    // group results of this round's fragments into the park area
#pragma unroll
    for (int f = 0; f < kChainFrag; ++f) {
      const int j = f / gpw, q = f - j * gpw;
      const int g = wave + kChainWaves * q;
      if (j < tn && g < G) {
        f32x4_t t[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const f32x4_t o = KEEP_OFF ? off[KEEP_OFF ? q : 0][ct] : group_offset(xa[q][ct]);
          t[ct] = NR == 1 ? f32x4_t{o[0], 0.0f, 0.0f, 0.0f} : o;
        }
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
            t[ct] = mfma16(xa[q][ct][d], PRE ? bw[PRE ? f : 0][d] : decode_nibbles<PACKED>(wf[f][d]),
                           t[ct]);
        const size_t pg = static_cast<size_t>(j) * G + g;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          if constexpr (NR == 1)
            tmps[(pg * CT + ct) * 64 + lane] = t[ct][0];
          else
            tmps[(pg * CT + ct) * 64 + lane] = t[ct];
        }
      }
    }
    __syncthreads();
    // tile t0 + wave: the canonical chain over the parked group results
    const int j = wave;
    auto tile_total = [&](f32x4_t (&total)[CT]) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) total[ct] = zero;
      for (int u = 0; u < U; ++u) {
        f32x4_t p[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) p[ct] = zero;
        const int gend = min(G, (u + 1) * kUnit);
        for (int g = u * kUnit; g < gend; ++g) {
          const size_t pg = static_cast<size_t>(j) * G + g;
          const float sc = scs[pg * 16 + i];
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            f32x4_t tv;
            if constexpr (NR == 1)
              tv = f32x4_t{tmps[(pg * CT + ct) * 64 + lane], 0.0f, 0.0f, 0.0f};
            else
              tv = tmps[(pg * CT + ct) * 64 + lane];
#pragma unroll
            for (int r = 0; r < NR; ++r) p[ct][r] = __builtin_fmaf(sc, tv[r], p[ct][r]);
          }
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) total[ct] = total[ct] + p[ct];
      }
    };
    // y bits of output row m, column n of projection v; a NaN sum (infinite
    // or NaN activations, overflow) is recomputed by the reference loop,
    // keeping its semantics
    auto out_bits = [&](float sum, const StageProj& v, int n, int m) -> uint32_t {
      float val = 16.0f * sum;
      if (__builtin_expect(val != val, 0))
        val = w4a16_ref_dot<PACKED, false, true>(v.w, v.s, K, n, S.x + static_cast<size_t>(m) * K);
      return f32_to_bf16_rne(val);
    };
    if (!epi) {
      if (wave < tn) {
        f32x4_t total[CT];
        tile_total(total);
        const int t = t0 + j;
        const StageProj v = stage_proj(S, t, epi);
        const int Nj = v.n;
        const int n = (t - v.begin) * kTileRows + i;
        if (n < Nj) {
          uint16_t* col = v.y + n;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int r = 0; r < NR; ++r) {
              const int m = ct * 16 + 4 * a + r;
              if (m < M)
                st_dev_u16(col + static_cast<size_t>(m) * Nj,
                           static_cast<uint16_t>(out_bits(total[ct][r], v, n, m)));
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete
      }
    } else {
      // SwiGLU: the up wave (odd j) of each pair parks its bf16 outputs
      // while the gate wave (even j) rounds silu(g); then the gate wave
      // writes act = silu(g) * up
      f32x4_t total[CT];
      if (wave < tn) tile_total(total);
      const int t = t0 + j;
      const StageProj v = stage_proj(S, t, epi);
      const int Nj = v.n;
      const int n = (t - v.begin) * kTileRows + i;
      uint32_t* px = xch + static_cast<size_t>(j >> 1) * CT * NR * 64;
      uint32_t sb[CT][NR];
      if (wave < tn && n < Nj) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const int m = ct * 16 + 4 * a + r;
            if (m < M) {
              const uint32_t o = out_bits(total[ct][r], v, n, m);
              if (j & 1)
                px[(ct * NR + r) * 64 + lane] = o;
              else
                sb[ct][r] = silu_bits(o);
            }
          }
      }
      __syncthreads();
      if (wave < tn && !(j & 1) && n < Nj) {
        uint16_t* col = S.act + n;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const int m = ct * 16 + 4 * a + r;
            if (m < M)
              st_dev_u16(col + static_cast<size_t>(m) * Nj,
                         static_cast<uint16_t>(mul_bits(sb[ct][r], px[(ct * NR + r) * 64 + lane])));
          }
      }
      __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete
    }
    __syncthreads();  // every store of the round is complete; the park area is free
  }
}

template <bool PACKED, int NR, int CT>
__global__ __launch_bounds__(kChainWaves * 64) void w4a16_chain_kernel(
    const ChainStage* __restrict__ table, uint32_t* __restrict__ flags, uint8_t* __restrict__ hdr,
    int nst, int M, int gt_max) {
  // The stage table is read-only for the launch and passed apart from the
  // words the launch writes, so its fields are wave-uniform scalar loads.
  // dynamic LDS only (a static variable would count against the 160 KB the
  // large-LDS opt-in grants): the park area
  extern __shared__ f32x4_t lds_park[];
  uint32_t* err = reinterpret_cast<uint32_t*>(hdr + kErrorOff);
  const int nwgs = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  // this launch's epoch: the workgroup's own epoch word + 1 (every
  // workgroup of the fixed grid runs every launch, so all words advance
  // together and the workgroups agree on it)
  // together and the workgroups agree on it). Every lane loads the two
  // words and keeps them in registers: they are first used at the first
  // wait or flag store, and loads complete in issue order, so the first
  // stage's weight loads are not held behind these round trips.
  uint32_t* my_epoch = reinterpret_cast<uint32_t*>(hdr + kEpochsOff) + blockIdx.x;
  const uint32_t e = ld_dev_u32(my_epoch) + 1u;
  const uint32_t bound = ld_dev_u32(reinterpret_cast<uint32_t*>(hdr + kBoundOff));
  const uint32_t ticks = bound != 0 ? bound : kDefaultWaitTicks;

  for (int s = 0; s < nst; ++s) {
    const ChainStage& S = table[s];
    int slot = b - S.first;
    if (slot < 0) slot += nwgs;
    if (slot >= S.nwg) continue;
    const int G = S.K >> 7;
    if (G <= kChainWaves)
      chain_stage<PACKED, NR, CT, 1>(S, slot, M, gt_max, lds_park, flags, e, err, ticks);
    else if (G <= 2 * kChainWaves)
      chain_stage<PACKED, NR, CT, 2>(S, slot, M, gt_max, lds_park, flags, e, err, ticks);
    else
      chain_stage<PACKED, NR, CT, 4>(S, slot, M, gt_max, lds_park, flags, e, err, ticks);
    if (threadIdx.x == 0) st_dev_u32(flags + (s * kChainFlagSlots + slot) * kChainFlagStride, e);
  }

  // the next launch of the chain starts from this one's epoch
  if (threadIdx.x == 0) st_dev_u32(my_epoch, e);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// Groups per wave of a stage's kernel path (1, 2 or 4).
int chain_gpw(int G) { return G <= kChainWaves ? 1 : G <= 2 * kChainWaves ? 2 : 4; }

// Occupancy query (grid == nullptr) or launch of one kernel instance.
template <bool PACKED, int NR, int CT>
int chain_launch_t(uint8_t* ws, int nst, int M, int gt, int* grid_or_occ, bool launch,
                   hipStream_t stream) {
  auto kern = w4a16_chain_kernel<PACKED, NR, CT>;
  const size_t lds = chain_lds_bytes(M, gt);
  if (!allow_lds(kern, lds)) return CUDALM_W4A16_ELAUNCH;
  if (!launch) {
    // resident workgroups per CU: registers (512 per SIMD lane, allocated
    // in blocks of 8; 8 waves = 2 per SIMD per workgroup) and LDS
    const int regs = regs_of(kern);
    if (regs <= 0) return CUDALM_W4A16_ELAUNCH;
    const int waves_per_simd = std::min(8, 512 / ((regs + 7) / 8 * 8));
    const int by_regs = waves_per_simd * 4 / kChainWaves;
    const int by_lds = static_cast<int>(kLdsMax / (lds + 64));
    *grid_or_occ = std::min(by_regs, by_lds);
    return CUDALM_W4A16_OK;
  }
  const ChainStage* table = reinterpret_cast<const ChainStage*>(ws + kChainHeader);
  uint32_t* flags = reinterpret_cast<uint32_t*>(ws + kChainHeader + chain_table_bytes(nst));
  hipLaunchKernelGGL(kern, dim3(*grid_or_occ), dim3(kChainWaves * 64), lds, stream, table, flags, ws,
                     nst, M, gt);
  return launch_status();
}

int chain_launch(int prepacked, uint8_t* ws, int nst, int M, int gt, int* grid_or_occ, bool launch,
                 hipStream_t stream) {
  if (prepacked) {
    if (M == 1) return chain_launch_t<true, 1, 1>(ws, nst, M, gt, grid_or_occ, launch, stream);
    if (M <= 16) return chain_launch_t<true, 4, 1>(ws, nst, M, gt, grid_or_occ, launch, stream);
    return chain_launch_t<true, 4, 2>(ws, nst, M, gt, grid_or_occ, launch, stream);
  }
  if (M == 1) return chain_launch_t<false, 1, 1>(ws, nst, M, gt, grid_or_occ, launch, stream);
  if (M <= 16) return chain_launch_t<false, 4, 1>(ws, nst, M, gt, grid_or_occ, launch, stream);
  return chain_launch_t<false, 4, 2>(ws, nst, M, gt, grid_or_occ, launch, stream);
}

int chain_plan_into(const cudalm_w4a16_stage* stages, int n_stages, int M, int prepacked,
                    void* workspace, size_t workspace_bytes, cudalm_w4a16_chain* chain,
                    hipStream_t stream, ChainStage* tab);

}  // namespace

extern "C" {

size_t cudalm_w4a16_chain_workspace_bytes(int n_stages) {
  if (n_stages < 1 || n_stages > CUDALM_W4A16_MAX_STAGES) return 0;
  return kChainHeader + chain_table_bytes(n_stages) + chain_flag_bytes(n_stages);
}

int cudalm_w4a16_chain_plan(const cudalm_w4a16_stage* stages, int n_stages, int M, int prepacked,
                            void* workspace, size_t workspace_bytes, cudalm_w4a16_chain* chain,
                            hipStream_t stream) {
  if (n_stages < 1 || n_stages > CUDALM_W4A16_MAX_STAGES) return CUDALM_W4A16_EINVAL;
  std::vector<ChainStage> tab(static_cast<size_t>(n_stages));
  return chain_plan_into(stages, n_stages, M, prepacked, workspace, workspace_bytes, chain, stream,
                         tab.data());
}

}  // extern "C"

namespace {

// Allocation-free chains (cudalm_w4a16_gemv_bf16_chain_noalloc): the plan,
// flags and counters live in this file-scope device array, one copy per
// GPU, up to kChainStaticStages stages. Host code never uses the array's
// name as an address: the device address comes from hipGetSymbolAddress,
// looked up once per device with that device current, and is what every
// copy, memset and kernel argument uses.
constexpr int kChainStaticStages = 128;
constexpr size_t kChainStaticBytes =
    kChainHeader + static_cast<size_t>(kChainStaticStages) * sizeof(ChainStage) +
    static_cast<size_t>(kChainStaticStages) * kChainFlagSlots * kChainFlagStride * 4;
static __device__ __align__(256) uint8_t scratch[kChainStaticBytes];

void* scratch_ptr() {
  static std::atomic<void*> ptrs[kMaxDevices];
  const int dev = current_device();
  if (dev < 0) return nullptr;
  void* p = ptrs[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return nullptr;
    ptrs[dev].store(p, std::memory_order_release);
  }
  return p;
}

// A stage's workgroups (nwg, at most max_wg) and tiles per workgroup and
// round (tpw, at most what the registers hold). A SwiGLU stage takes an
// even tpw (4 or 2 fit: K <= 2048), so every round holds whole pairs.
void chain_split(ChainStage& T, int M, int max_wg) {
  const int G = T.K / kGroup;
  const int tcap = chain_frag(chain_gpw(G), M > 16 ? 2 : 1) / chain_gpw(G);
  const int nwg = (T.ntiles + tcap - 1) / tcap;
  T.nwg = nwg < max_wg ? nwg : max_wg;
  T.tpw = (T.ntiles + T.nwg - 1) / T.nwg;
  if (T.act != nullptr) T.tpw = (T.tpw + 1) & ~1;
  if (T.tpw > tcap) T.tpw = tcap;
  if (T.act != nullptr) T.nwg = std::min(max_wg, (T.ntiles + T.tpw - 1) / T.tpw);
}

// The plan, written into `workspace` from the host table `tab` (n_stages
// entries, filled here).
int chain_plan_into(const cudalm_w4a16_stage* stages, int n_stages, int M, int prepacked,
                    void* workspace, size_t workspace_bytes, cudalm_w4a16_chain* chain,
                    hipStream_t stream, ChainStage* tab) {
  if (!stages || !workspace || !chain) return CUDALM_W4A16_ENULL;
  if (n_stages < 1 || n_stages > CUDALM_W4A16_MAX_STAGES || M < 1 || M > 32)
    return CUDALM_W4A16_EINVAL;
  const size_t need = cudalm_w4a16_chain_workspace_bytes(n_stages);
  if (workspace_bytes < need) return CUDALM_W4A16_EINVAL;
  if (!aligned(workspace, 256)) return CUDALM_W4A16_EALIGN;
  int gt_max = 0;  // max tpw * G over stages
  for (int s = 0; s < n_stages; ++s) {
    const cudalm_w4a16_stage& st = stages[s];
    ChainStage& T = tab[static_cast<size_t>(s)];
    memset(&T, 0, sizeof(T));
    if (st.count < 1 || st.count > kChainProj) return CUDALM_W4A16_EINVAL;
    if (!st.projs || !st.x) return CUDALM_W4A16_ENULL;
    if (st.K <= 0 || st.K % kGroup != 0 || st.K > kChainWaves * kChainGpw * kGroup)
      return CUDALM_W4A16_EINVAL;
    if (st.dep < -1 || st.dep >= s) return CUDALM_W4A16_EINVAL;
    if (!aligned(st.x, 16)) return CUDALM_W4A16_EALIGN;
    const bool epi = st.act != nullptr;
    if (epi) {
      // SwiGLU: gate and up of one shape, at most two groups per wave so a
      // round holds whole tile pairs
      if (st.count != 2 || st.projs[0].N != st.projs[1].N || st.K > 2 * kChainWaves * kGroup)
        return CUDALM_W4A16_EINVAL;
      if (!aligned(st.act, 2)) return CUDALM_W4A16_EALIGN;
    }
    int tiles = 0;
    for (int j = 0; j < st.count; ++j) {
      const cudalm_w4a16_proj& p = st.projs[j];
      if (p.N < 1 || p.N > (1 << 24)) return CUDALM_W4A16_EINVAL;
      if (!p.weight || (!epi && !p.y) || (!prepacked && !p.scale)) return CUDALM_W4A16_ENULL;
      if (!aligned(p.weight, 16) || (!epi && !aligned(p.y, 2)) ||
          (!prepacked && !aligned(p.scale, 2)))
        return CUDALM_W4A16_EALIGN;
      T.w[j] = static_cast<const uint8_t*>(p.weight);
      T.s[j] = p.scale;
      T.y[j] = p.y;
      T.n[j] = p.N;
      tiles += (p.N + kTileRows - 1) / kTileRows;
      T.tile_end[j] = tiles;
    }
    if (static_cast<long long>(M) * st.K > (1LL << 30)) return CUDALM_W4A16_ERANGE;
    T.x = st.x;
    T.act = st.act;
    T.count = st.count;
    T.K = st.K;
    T.dep = st.dep;
    T.ntiles = tiles;
    chain_split(T, M, kChainMaxWg);
    if (T.tpw * (st.K / kGroup) > gt_max) gt_max = T.tpw * (st.K / kGroup);
  }
  int occ = 0;
  if (int rc = chain_launch(prepacked, nullptr, n_stages, M, gt_max, &occ, false, stream)) return rc;
  if (occ < 1) return CUDALM_W4A16_ELAUNCH;
  const int grid = std::min(cu_count() * occ, kChainMaxGrid);
  int first = 0;
  for (int s = 0; s < n_stages; ++s) {
    ChainStage& T = tab[static_cast<size_t>(s)];
    if (T.nwg > grid) chain_split(T, M, grid);  // fewer resident workgroups: more rounds
    T.first = first;
    first = (first + T.nwg) % grid;
    T.dep_nwg = T.dep >= 0 ? tab[static_cast<size_t>(T.dep)].nwg : 0;
  }
  // header and flags zeroed, then the stage table
  if (hipMemsetAsync(workspace, 0, need, stream) != hipSuccess) return CUDALM_W4A16_ELAUNCH;
  if (hipMemcpyAsync(static_cast<uint8_t*>(workspace) + kChainHeader, tab,
                     chain_table_bytes(n_stages), hipMemcpyHostToDevice, stream) != hipSuccess)
    return CUDALM_W4A16_ELAUNCH;
  if (hipStreamSynchronize(stream) != hipSuccess) return CUDALM_W4A16_ELAUNCH;
  chain->workspace = workspace;
  chain->n_stages = n_stages;
  chain->M = M;
  chain->prepacked = prepacked ? 1 : 0;
  chain->grid = grid;
  chain->gt_max = gt_max;
  return CUDALM_W4A16_OK;
}

}  // namespace

extern "C" {

int cudalm_w4a16_chain_run(const cudalm_w4a16_chain* chain, hipStream_t stream) {
  if (!chain || !chain->workspace) return CUDALM_W4A16_ENULL;
  if (chain->n_stages < 1 || chain->n_stages > CUDALM_W4A16_MAX_STAGES || chain->M < 1 ||
      chain->M > 32 || chain->grid < 1)
    return CUDALM_W4A16_EINVAL;
  int grid = chain->grid;
  return chain_launch(chain->prepacked, static_cast<uint8_t*>(chain->workspace), chain->n_stages,
                      chain->M, chain->gt_max, &grid, true, stream);
}

int cudalm_w4a16_chain_status(const cudalm_w4a16_chain* chain, hipStream_t stream) {
  if (!chain || !chain->workspace) return CUDALM_W4A16_ENULL;
  if (hipStreamSynchronize(stream) != hipSuccess) return CUDALM_W4A16_ELAUNCH;
  uint32_t word = 0;
  uint8_t* errp = static_cast<uint8_t*>(chain->workspace) + kErrorOff;
  if (hipMemcpy(&word, errp, sizeof(word), hipMemcpyDeviceToHost) != hipSuccess)
    return CUDALM_W4A16_ELAUNCH;
  if (word == 0) return CUDALM_W4A16_OK;
  if (hipMemset(errp, 0, sizeof(word)) != hipSuccess) return CUDALM_W4A16_ELAUNCH;
  return CUDALM_W4A16_ETIMEOUT;
}

int cudalm_w4a16_chain_set_wait_bound(const cudalm_w4a16_chain* chain, uint32_t ticks,
                                      hipStream_t stream) {
  if (!chain || !chain->workspace) return CUDALM_W4A16_ENULL;
  uint8_t* bp = static_cast<uint8_t*>(chain->workspace) + kBoundOff;
  if (hipMemcpyAsync(bp, &ticks, sizeof(ticks), hipMemcpyHostToDevice, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return CUDALM_W4A16_ELAUNCH;
  return CUDALM_W4A16_OK;
}

int cudalm_w4a16_gemv_bf16_chain(const cudalm_w4a16_stage* stages, int n_stages, int M,
                                 int prepacked, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  cudalm_w4a16_chain chain;
  if (int rc = cudalm_w4a16_chain_plan(stages, n_stages, M, prepacked, workspace, workspace_bytes,
                                       &chain, stream))
    return rc;
  return cudalm_w4a16_chain_run(&chain, stream);
}

int cudalm_w4a16_gemv_bf16_chain_noalloc(const cudalm_w4a16_stage* stages, int n_stages, int M,
                                         int prepacked, hipStream_t stream) {
  if (n_stages > kChainStaticStages) return CUDALM_W4A16_ERANGE;
  if (n_stages < 1) return CUDALM_W4A16_EINVAL;
  void* ws = scratch_ptr();
  if (ws == nullptr) return CUDALM_W4A16_ELAUNCH;
  ChainStage tab[kChainStaticStages];  // host copy of the plan, on the stack
  cudalm_w4a16_chain chain;
  if (int rc = chain_plan_into(stages, n_stages, M, prepacked, ws, kChainStaticBytes, &chain, stream,
                               tab))
    return rc;
  return cudalm_w4a16_chain_run(&chain, stream);
}

}  // extern "C"
