// Paged prefill / chunked-prefill attention for gfx950: MFMA tiles over K/V staged in LDS.
//
// The same arithmetic as `LayerPass::attend` (crates/yaxus-backend-cpu/src/lib.rs:
// 389-427) for passes with many rows per sequence, the shape the reference's tiled
// kernel serves (ATTN_TILE, crates/yaxus-backend-gpu/src/shaders.rs:422-592: 32 rows x
// 32-key blocks, f32 SIMT). Here a workgroup of 4 waves (one per SIMD) takes a tile of
// kPrefillRows = 64 logical rows, the (row, query head) pairs of consecutive rows of one
// sequence and one KV head; each wave owns 16 of them, the 16 columns of its MFMA tile.
// Keys stream from HBM straight into a 4-slot LDS ring of 32-key stages (64 KiB;
// global_load_lds_dwordx4, no registers; two stages in flight), and every wave reads
// them there. Two workgroups share a CU (two waves per SIMD, at most 256 registers each)
// and run out of phase, so one's start, barriers and output overlap the other's
// products (cfg3: 86-87 us against 90-91 with one 8-wave workgroup of 128 rows and a
// 128 KiB ring of 64-key stages per CU). Per 32 keys:
//   S^T[key][row] = K . Q^T      8 x v_mfma_f32_16x16x32_f16 per tile (q as hi + lo f16)
//   online softmax per column, once per 32 keys (permlane swaps across lane groups);
//   the accumulator is rescaled only when a column's maximum grew by more than
//   kLazyRescale
//   O^T += V^T P^T               16 x v_mfma_f32_16x16x32_f16 per tile (P hi + lo)
// q and P each go in as a binary16 hi part plus a lo part, two products into one
// result, so both keep ~2^-22 relative accuracy (a single rounding of P costs up to
// 5e-4 absolute against the f32 oracle, 1.3e-3 with q three times larger); K and V are
// binary16 already. This doubles the MFMA work of the plain-f16 form. The tests compare
// with the f32 oracle and an f64 brute force. Key pairs no column of a wave can see
// (causal, window) are skipped by that wave. When a pass has too few tiles for the GPU
// (one sequence's chunk after a long context), the host splits tiles along keys: each
// chunk is its own work item, writes its columns' partial softmax, and the tile's last
// chunk merges them in chunk order (merge_tile; the hand-off of the split-K decode
// kernels).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_decode.hpp"

namespace yx {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_raw __attribute__((__vector_size__(8)));  // the builtin's operand type
typedef __attribute__((address_space(3))) fp16x4_raw lds_half4;

struct PrefillItem {
  uint32_t r0;      // first pass row of the tile
  uint32_t nrows;   // rows (positions) in the tile
  uint32_t pt_off;  // the sequence's page table in the pass's pages
  uint32_t blk0;    // first key block of this item's key range
  uint32_t blk1;    // one past its last key block
  // A tile whose keys are split over several items (a long context and too few tiles to
  // fill the GPU): chunk index in bits 0-15, chunk count in bits 16-31 (1: not split).
  uint32_t chunk_nch;
  uint32_t part_base;  // partial slot of chunk 0 (split tiles)
  uint32_t counter;    // arrival counter of the tile (split tiles)
};

// Merges a split tile's chunks (the tile's last chunk does it): the partial (maximum,
// sum, unnormalised O) of each logical row in chunk slots base .. base + nch - 1, in
// chunk order, so the result does not depend on arrival order. A thread takes kPer
// (row, 4 dims) entries, kGE at a time, and has the loads of kCB chunks of those kGE
// entries in flight at once (a tile's partials are many: 64 or 128 rows per chunk).
template <int kThreads, int kRows>
__device__ __forceinline__ void merge_tile(uint32_t r0, uint32_t nrows, uint32_t base, uint32_t nch,
                                           uint32_t kh, uint32_t G, uint32_t hq, uint32_t hkv,
                                           float* __restrict__ out, __amdgpu_buffer_rsrc_t ro,
                                           __amdgpu_buffer_rsrc_t rml) {
  constexpr int kPer = kRows * 32 / kThreads;
  constexpr int kGE = 4, kCB = 4;
  static_assert(kPer % kGE == 0, "whole groups of entries per thread");
  const uint32_t nlog = nrows * G;
  const size_t qd = static_cast<size_t>(hq) * kD;
#pragma unroll
  for (int e0 = 0; e0 < kPer; e0 += kGE) {
    float mt[kGE], lt[kGE];
    float4 o[kGE];
    uint32_t lr[kGE], qi[kGE];
#pragma unroll
    for (int j = 0; j < kGE; ++j) {
      const uint32_t idx = threadIdx.x + (e0 + j) * kThreads;
      lr[j] = idx >> 5;
      qi[j] = idx & 31;
      mt[j] = -INFINITY;
      lt[j] = 0.0f;
      o[j] = float4{0, 0, 0, 0};
    }
    for (uint32_t c0 = 0; c0 < nch; c0 += kCB) {
      float2 ml[kGE][kCB];
      float4 po[kGE][kCB];
#pragma unroll
      for (int j = 0; j < kGE; ++j)
#pragma unroll
        for (int b = 0; b < kCB; ++b) {
          const uint32_t ch = min(c0 + b, nch - 1);
          const size_t e = ((static_cast<size_t>(base) + ch) * hkv + kh) * kRows + (lr[j] < nlog ? lr[j] : 0u);
          ml[j][b] = ld2_coherent(rml, static_cast<uint32_t>(e * 8));
          po[j][b] = ld4_coherent(ro, static_cast<uint32_t>((e * kD + qi[j] * 4) * 4));
        }
#pragma unroll
      for (int j = 0; j < kGE; ++j)
#pragma unroll
        for (int b = 0; b < kCB; ++b) {
          if (c0 + b >= nch || !(ml[j][b].y > 0.0f)) continue;  // past the list, or empty
          const float mn = fmaxf(mt[j], ml[j][b].x);
          const float r = __builtin_amdgcn_exp2f(mt[j] - mn), wt = __builtin_amdgcn_exp2f(ml[j][b].x - mn);
          lt[j] = lt[j] * r + ml[j][b].y * wt;
          o[j] = float4{o[j].x * r + po[j][b].x * wt, o[j].y * r + po[j][b].y * wt,
                        o[j].z * r + po[j][b].z * wt, o[j].w * r + po[j][b].w * wt};
          mt[j] = mn;
        }
    }
#pragma unroll
    for (int j = 0; j < kGE; ++j) {
      if (lr[j] >= nlog) continue;
      const uint32_t rr = r0 + lr[j] / G, h = kh * G + lr[j] % G;
      const float inv = 1.0f / lt[j];
      *reinterpret_cast<float4*>(out + rr * qd + h * kD + qi[j] * 4) =
          float4{o[j].x * inv, o[j].y * inv, o[j].z * inv, o[j].w * inv};
    }
  }
}

#ifdef YX_PF_PROF
// Phase clocks of the prefill kernel, summed over waves (a profiling build only).
// Slot [k][wave of the launch], overwritten by each launch.
__device__ unsigned long long g_pf_prof[16][16384];
#define PF_NOW() __builtin_amdgcn_s_memtime()
#define PF_CYC(v) const uint64_t v = __builtin_amdgcn_s_memtime()
#define PF_ACC(a, x, y) a += ((y) - (x))
#define PF_ADD(k, v) \
  if ((threadIdx.x & 63) == 0 && blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6) < 16384u) \
    g_pf_prof[k][blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = static_cast<unsigned long long>(v)
#else
#define PF_NOW() 0ull
#define PF_ADD(k, v)
#define PF_CYC(v)
#define PF_ACC(a, x, y)
#endif

static constexpr int kPrefillWaves = 4;
static constexpr int kPrefillTiles = 1;  // MFMA tiles (16 logical rows) per wave
static constexpr int kPrefillRows = kPrefillWaves * kPrefillTiles * 16;  // logical rows per item

static constexpr int kStageBlocks = 2;  // 16-key blocks per LDS stage (32 keys, 16 KiB of K+V)
static constexpr int kRing = 4;  // LDS stages: kLead in flight, one computed, one finishing
static constexpr int kLead = kRing - 2;
static constexpr float kLazyRescale = 8.0f;    // log2 headroom before the maximum moves

// One 16-byte piece per lane from global memory straight into LDS (no registers): lane
// i's piece lands at LDS byte address `lds` + 16 i. M0 holds the wave's LDS base for
// the instruction and is restored afterwards. The load counts in vmcnt like any other;
// callers wait for it explicitly (the compiler does not know about it).
__device__ __forceinline__ void load_to_lds16(const void* src, uint32_t lds) {
  uint32_t saved;
  __asm__ volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(lds)
      : "memory");
}

// Keeps a value's computation at this point of the instruction stream: the empty asm
// consumes and redefines the register, so the arithmetic that produces it cannot be sunk
// past here (towards its first real use) by the compiler's code motion. The pair step
// below uses it to keep its softmax slices between the matrix products they are meant to
// overlap with.
template <typename T>
__device__ __forceinline__ void pin(T& v) {
  __asm__ volatile("" : "+v"(v));
}

// max(a, b, c) in one instruction (fmaxf would first quiet each MFMA result with a
// self-max of its own; scores are never signalling NaNs).
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  __asm__("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// One block half (4 KiB: 4 rows of 1 KiB) from global memory straight into LDS: row r
// comes from base + off[r % 2] + 1024 r (the lanes' 16-byte pieces) and lands at LDS
// byte address lds + 1024 r (lane i's piece at + 16 i). The global address is the
// scalar base plus a 32-bit lane offset; the instruction's immediate offset applies to
// both the global and the LDS address, so M0 (the LDS address) is set once for the four
// rows (its previous value is restored after). The loads count in vmcnt like any other;
// callers wait for them explicitly (the compiler does not know about them).
__device__ __forceinline__ void load_half_to_lds(const void* base, uint32_t off0, uint32_t off1, uint32_t lds) {
  uint32_t saved;  // M0 is the compiler's
  __asm__ volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %4\n\t"
      "global_load_lds_dwordx4 %2, %1\n\t"
      "global_load_lds_dwordx4 %3, %1 offset:1024\n\t"
      "global_load_lds_dwordx4 %2, %1 offset:2048\n\t"
      "global_load_lds_dwordx4 %3, %1 offset:3072\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(base), "v"(off0), "v"(off1), "s"(lds)
      : "memory");
}

// W waves of NT MFMA tiles each (W * NT * 16 = kPrefillRows logical rows) over stages of
// SBT blocks; 8 / W waves per SIMD (an 8-wave workgroup fills a CU; two 4-wave ones share
// it). Each wave overlaps its own matrix products with its softmax arithmetic
// (software-pipelined below).
// QKV: q is not given; the kernel reads its rows' raw q heads from qkv and normalises
// and rotates them itself, with write_rows' arithmetic (the same bits as
// qk_norm_rope_append), the key heads having been stored before the launch.
template <bool QKV, int W = kPrefillWaves, int NT = kPrefillTiles, int SBT = kStageBlocks>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(8 / W, 8 / W))) void paged_attn_prefill(
    const PrefillItem* __restrict__ items, const uint32_t* pos,
    const uint32_t* __restrict__ pages, const _Float16* __restrict__ kc,
    const _Float16* __restrict__ vc, const float* q, float* __restrict__ out,
    uint32_t hq, uint32_t hkv, uint32_t bpp_shift, uint32_t window, float scale_log2,
    QkvIn qi_in, float* __restrict__ part_o, float2* __restrict__ part_ml,
    uint32_t* __restrict__ counters, uint32_t part_o_bytes, uint32_t part_ml_bytes) {
  constexpr int SB = SBT;
  static_assert(SB == 2 || SB == 4, "stages of one or two pairs of blocks");
  constexpr int PPS = SB / 2;  // pairs of 16-key blocks per stage
  static_assert(W * NT * 16 == kPrefillRows, "a work item's rows are W waves of NT tiles");
  // A ring of stages; each holds SB blocks of K as [p][g][key] (4 KiB each) and then SB
  // blocks of V as [key][128] (4 KiB each).
  __shared__ half8 ring[kRing][2 * SB * 256];
  // One dimension, KV head fastest: workgroups start in the host's longest-first item
  // order across all KV heads.
  const uint64_t pf_t0 = PF_NOW();
#ifdef YX_PF_PROF
  const uint64_t pf_r0 = __builtin_amdgcn_s_memrealtime();
#endif
  uint64_t pf_stage = 0, pf_rare = 0, pf_b0 = 0, pf_b1 = 0, pf_b2 = 0, pf_b3 = 0;
  (void)pf_t0; (void)pf_stage; (void)pf_rare;
  const PrefillItem it = items[blockIdx.x / hkv];
  const uint32_t kh = blockIdx.x % hkv;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const uint32_t G = hq / hkv;
  const uint32_t nlog = it.nrows * G;

  const uint32_t bpp_mask = (1u << bpp_shift) - 1u;
  const size_t head_stride = static_cast<size_t>(16u << bpp_shift) * kD;
  const uint32_t* pt = pages + it.pt_off;
  // Each wave moves HW of the stage's 2 * SB block halves, half h being block h / 2's K
  // (h even) or V (h odd), as four 1 KiB rows each. K row p is read transposed ([p][key][g]
  // in the arena, [p][g][key] in LDS): lane l fetches key l % 16, dims group l / 16. V
  // keeps its [key][128] rows, but the 32-byte chunks of key k's row are stored
  // XOR-swizzled (chunk j at j ^ (k & 7)) so that the transposing reads below stay at the
  // minimum of two passes per 512 bytes; within a 1 KiB row lane l lands on key
  // 4 r + l / 16, piece l % 16, and so fetches the piece that belongs there.
  static_assert((2 * SB) % W == 0, "whole block halves per wave");
  constexpr int HW = 2 * SB / W;
  constexpr int kRowsPerWave = 4 * HW;  // 1 KiB rows (loads) per wave per stage
  // Lane offsets of rows r = 0, 1 (rows 2 and 3 repeat them 2 KiB on).
  uint32_t src_k[2], src_v[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint32_t key = 4 * r + (lane >> 4), pp = lane & 15;
    src_v[r] = key * 256u + (2u * ((pp >> 1) ^ (key & 7u)) + (pp & 1u)) * 16u;
    src_k[r] = static_cast<uint32_t>(r * 1024 + ((lane & 15) * 4 + (lane >> 4)) * 16);
  }
  const uint32_t ring_base = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) half8*)&ring[0][0]));
  // The page ids of the block this wave moves, from an LDS table of two 64-stage batches
  // per wave (lane l of a batch's load fetches stage 64 k + l's id straight into the
  // table): batches 0 and 1 are loaded at the start, batch k + 1 when batch k comes into
  // use, 64 stages before it is read. The loads count in vmcnt and are complete long
  // before they are read (the stages' own waits pass them). Stages 0 and 1 take their ids
  // from a scalar read of the page table; each later stage reads its id from the table one
  // stage ahead, so the loop never waits for a page-table read in memory.
  static_assert(HW == 1, "one block half per wave and stage");
  __shared__ uint32_t pid_tab[W][2][64];
  const uint32_t my_blk = static_cast<uint32_t>(wave >> 1);
  const bool my_v = (wave & 1) != 0;
  auto block_of = [&](uint32_t st) __attribute__((always_inline)) {  // past the end: the last block (unused)
    const uint32_t b = it.blk0 + st * SB + my_blk;
    return b < it.blk1 ? b : it.blk1 - 1;
  };
  const uint32_t tab_base = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint32_t*)&pid_tab[wave][0][0]));
  auto load_batch = [&](uint32_t k) __attribute__((always_inline)) {
    const uint32_t* src = pt + (block_of(64u * k + static_cast<uint32_t>(lane)) >> bpp_shift);
    uint32_t saved;
    __asm__ volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dword %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(tab_base + (k & 1u) * 256u)
        : "memory");
  };
  auto tab_read = [&](uint32_t st) __attribute__((always_inline)) {
    return pid_tab[wave][(st >> 6) & 1u][st & 63u];
  };
  // This wave's half of every block: K or V, its KV head's part of each page.
  const char* const half_base = reinterpret_cast<const char*>(my_v ? vc : kc) + static_cast<size_t>(kh) * head_stride * 2;
  const uint32_t page_bytes = static_cast<uint32_t>(hkv * head_stride * 2);
  // Stages 0-2 take their ids from scalar reads of the page table, waited for at once (the
  // batches' loads are only known complete after the first stage's wait); each later
  // stage's id is read from the table during the stage before.
  auto pt_at = [&](uint32_t st) __attribute__((always_inline)) {
    return pt + __builtin_amdgcn_readfirstlane(block_of(st) >> bpp_shift);
  };
  uint32_t pid_pre;
  auto issue_page = [&](uint32_t st, uint32_t slot, uint32_t page) __attribute__((always_inline)) {
    const uint32_t blkin = block_of(st) & bpp_mask;
    const char* blk = half_base + static_cast<uint64_t>(page) * page_bytes + blkin * 4096u;
    const uint32_t dst = ring_base + slot * (2 * SB * 256 * 16) + (my_v ? SB * 4096u : 0u) + my_blk * 4096u;
    if (my_v)
      load_half_to_lds(blk, src_v[0], src_v[1] - 1024u, dst);
    else
      load_half_to_lds(blk, src_k[0], src_k[1] - 1024u, dst);
  };
  auto issue = [&](uint32_t st, uint32_t slot) __attribute__((always_inline)) {  // stage st >= 2 into ring slot `slot`
    const uint32_t page = __builtin_amdgcn_readfirstlane(pid_pre);
    if ((st & 63u) == 0) load_batch(st / 64u + 1u);  // wave-uniform, once per 64 stages
    pid_pre = tab_read(st + 1);
    issue_page(st, slot, page);
  };
  load_batch(0);
  load_batch(1);
  // q and pos are read first, unconditionally (rows past the tile read row 0 and are
  // zeroed), so that waiting for them does not wait for the K/V stages issued after.
  // q and pos are not declared __restrict__ and the empty asm may write memory, so the
  // compiler cannot sink these loads below the stage loads.
  float4 qraw[NT][8];
  int rpos[NT], rlo[NT];
  uint32_t rowp[NT];  // the column's position (row 0's for an empty column)
  bool has[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint32_t lr = (wave * NT + t) * 16 + c;
    has[t] = lr < nlog;
    const uint32_t lrc = has[t] ? lr : 0;
    const uint32_t rr = it.r0 + lrc / G, h = kh * G + lrc % G;
    const int p = static_cast<int>(pos[rr]);
    rpos[t] = has[t] ? p : -1;
    rlo[t] = (window > 0 && p + 1 > static_cast<int>(window)) ? p + 1 - static_cast<int>(window) : 0;
    rowp[t] = p;
    const float* qp = QKV ? qi_in.qkv + static_cast<size_t>(rr) * (hq + 2 * hkv) * kD + h * kD + g * 8
                          : q + (static_cast<size_t>(rr) * hq + h) * kD + g * 8;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      qraw[t][2 * pp] = *reinterpret_cast<const float4*>(qp + pp * 32);
      qraw[t][2 * pp + 1] = *reinterpret_cast<const float4*>(qp + pp * 32 + 4);
    }
  }
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t nst = (it.blk1 - it.blk0 + SB - 1) / SB;  // stages
  static_assert(kLead == 2, "stages 0 and 1 are issued first");
  {
    uint32_t p0, p1;
    __asm__ volatile(
        "s_load_dword %0, %3, 0x0\n\t"
        "s_load_dword %1, %4, 0x0\n\t"
        "s_load_dword %2, %5, 0x0\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(p0), "=&s"(p1), "=&s"(pid_pre)
        : "s"(pt_at(0)), "s"(pt_at(1)), "s"(pt_at(2))
        : "memory");
    issue_page(0, 0, p0);
    if (nst > 1) issue_page(1, 1, p1);
  }

  if constexpr (QKV) {
    // write_rows for the columns' q heads. Lane g of a column holds dims
    // 32 pp + 8 g + e; the sum of squares runs over dims 0..127 in order, so it passes
    // from lane group to lane group every 8 dims (the owner adds, all take its sum).
#pragma clang fp contract(off)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float x[32];
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const float4 a = qraw[t][2 * pp], b = qraw[t][2 * pp + 1];
        x[8 * pp] = a.x; x[8 * pp + 1] = a.y; x[8 * pp + 2] = a.z; x[8 * pp + 3] = a.w;
        x[8 * pp + 4] = b.x; x[8 * pp + 5] = b.y; x[8 * pp + 6] = b.z; x[8 * pp + 7] = b.w;
      }
      float ss = 0.0f;
#pragma unroll
      for (int s8 = 0; s8 < 16; ++s8) {
        const int pp = s8 >> 2, owner = s8 & 3;
        float cand = ss;
#pragma unroll
        for (int e = 0; e < 8; ++e) cand = cand + x[8 * pp + e] * x[8 * pp + e];
        ss = __shfl(cand, c + 16 * owner);
      }
      const float r = 1.0f / __builtin_sqrtf(ss / 128.0f + qi_in.eps);
      float y[32];
#pragma unroll
      for (int pp = 0; pp < 4; ++pp)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 32 * pp + 8 * g + e;
          y[8 * pp + e] = (1.0f + qi_in.q_norm[d]) * (x[8 * pp + e] * r);
        }
      const float* cs_row = qi_in.rope_cs + static_cast<size_t>(rowp[t]) * 64;
      const float* sn_row = qi_in.rope_cs + (static_cast<size_t>(qi_in.rope_len) + rowp[t]) * 64;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 32 * pp + 8 * g + e;  // dims j and j + 64 rotate together
          const float y0 = y[8 * pp + e], y1 = y[8 * (pp + 2) + e];
          const float cs = cs_row[j], sn = sn_row[j];
          const float ab = y0 * cs, bs = y1 * sn, bc = y1 * cs, as = y0 * sn;
          y[8 * pp + e] = ab - bs;
          y[8 * (pp + 2) + e] = bc + as;
        }
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        qraw[t][2 * pp] = float4{y[8 * pp], y[8 * pp + 1], y[8 * pp + 2], y[8 * pp + 3]};
        qraw[t][2 * pp + 1] = float4{y[8 * pp + 4], y[8 * pp + 5], y[8 * pp + 6], y[8 * pp + 7]};
      }
    }
  }
  half8 qh[NT][4], ql[NT][4];  // q as binary16 hi + lo parts
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const float4 a = qraw[t][2 * pp], b = qraw[t][2 * pp + 1];
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = has[t] ? x[e] * scale_log2 : 0.0f;  // scores come out in log2 units
        qh[t][pp][e] = static_cast<_Float16>(v);
        ql[t][pp][e] = static_cast<_Float16>(v - static_cast<float>(qh[t][pp][e]));
      }
    }
  // Uniform limits: per tile the last row's position, the first row's position and the
  // largest window start; per wave the key range any of its rows sees.
  int tmax[NT], tmin[NT], tlo[NT];
  int wmax = -1, wlo = INT32_MAX;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int mx = rpos[t], mn = rpos[t], lo = rpos[t] < 0 ? INT32_MAX : rlo[t], hl = rlo[t];
#pragma unroll
    for (int sft = 1; sft < 16; sft <<= 1) {
      mx = max(mx, __shfl_xor(mx, sft));
      mn = min(mn, __shfl_xor(mn, sft));
      lo = min(lo, __shfl_xor(lo, sft));
      hl = max(hl, __shfl_xor(hl, sft));
    }
    tmax[t] = __builtin_amdgcn_readfirstlane(mx);
    tmin[t] = __builtin_amdgcn_readfirstlane(mn);  // -1 when the tile has an empty column
    tlo[t] = __builtin_amdgcn_readfirstlane(hl);
    wmax = max(wmax, tmax[t]);
    wlo = min(wlo, __builtin_amdgcn_readfirstlane(lo));
  }

  // -FLT_MAX: the per-lane maximum of a pair whose keys are all masked (-inf); every
  // visible key's x is above it.
  constexpr float kNoKey = -3.40282347e38f;
  // Per column the running maximum m (log2 units of q.k / sqrt(d)), kept in the score
  // accumulators' starting value: the score MFMAs of a pair start from -m, so they return
  // x = s - m directly and the exponentials need no subtraction. A column that has seen
  // no key yet has m = 0 (its x are the raw scores, exact) and threshold thr = kNoKey, so
  // its first visible key triggers the (wave-uniform) move below; after that thr =
  // kLazyRescale: m moves only when some x exceeds it, so P = 2^x stays below
  // 2^kLazyRescale, well inside binary16 and f32, and the sum uses the same offset.
  float m[NT], thr[NT], lsum[NT];  // lsum: this lane's share of its column's sum (its 8 keys of every pair)
  floatx4 negm[NT];
  floatx4 acc[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m[t] = 0.0f;
    thr[t] = kNoKey;
    negm[t] = floatx4{0, 0, 0, 0};
    lsum[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[t][j] = floatx4{0, 0, 0, 0};
  }
  const int key_end = static_cast<int>(it.blk1 * 16);
  const int first_key = static_cast<int>(it.blk0 * 16);
  const int npair = static_cast<int>(PPS * nst);
  // Pair i holds keys first_key + 32 i .. + 31. This wave computes the pairs [pa, pb) that
  // hold a key some column of the wave can see; the others it only passes through.
  int pa = npair, pb = npair;
  if (wmax >= 0) {
    const int d = wlo - first_key;
    pa = d <= 0 ? 0 : d / 32;
    const int e = min(wmax, key_end - 1) - first_key;
    pb = e < 0 ? 0 : min(npair, e / 32 + 1);
  }
  // Whole pairs (every key visible to every column of the wave, no mask) are [wa, wb).
  int wtmin = INT32_MAX, wtlo = -1;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    wtmin = min(wtmin, tmin[t]);
    wtlo = max(wtlo, tlo[t]);
  }
  int wa = pa, wb = pa;
  if (pa < pb) {
    const int d = wtlo - first_key;
    wa = d <= 0 ? 0 : (d + 31) / 32;
    const int e = min(wtmin - 31, key_end - 32) - first_key;
    wb = e < 0 ? 0 : e / 32 + 1;
    wa = min(max(wa, pa), pb);
    wb = min(max(wb, wa), pb);
  }

  // Per lane, the byte offset of its transposing-read address for dim group j within a
  // block of V (see the swizzle above): key k = 4 g + c / 4, dims 16 j + 4 (c % 4).
  uint32_t vtr_off[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t k = 4u * g + (c >> 2);
    vtr_off[j] = k * 256u + 32u * (static_cast<uint32_t>(j) ^ (k & 7u)) + 8u * (c & 3);
  }

  // Stage st becomes readable: this wave's loads of it are done when at most the
  // kLead - 1 later stages' are in flight, and the barrier makes every wave's part
  // visible. Every wave has then also issued and (lgkmcnt) finished its reads of stage
  // st - 2, whose slot is refilled with stage st + kLead (the last pair of stage st - 1
  // still reads its V after the barrier). Stages past the item's last are not loaded, so
  // the last stage waits for every load, and the workgroup ends with none in flight.
#ifdef YX_PF_PROF
  uint64_t e0 = 0, e1 = 0, e2 = 0, e3 = 0, e4 = 0, pf_e1 = 0, pf_e2 = 0, pf_e3 = 0, pf_e4 = 0;
#endif
  auto stage_enter = [&](uint32_t st) __attribute__((always_inline)) {
#ifdef YX_PF_PROF
    e0 = PF_NOW();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    e1 = PF_NOW();
    if (st + 1 < nst)
      __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(kRowsPerWave * (kLead - 1)) : "memory");
    else
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    e2 = PF_NOW();
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    e3 = PF_NOW();
    if (st + kLead < nst) issue(st + kLead, (st + kLead) & (kRing - 1));
    e4 = PF_NOW();
#else
    if (st + 1 < nst)  // the next stage's loads may still be in flight
      __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)" ::"n"(kRowsPerWave * (kLead - 1))
                       : "memory");
    else  // the last stage: nothing was issued after it
      __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    if (st + kLead < nst) issue(st + kLead, (st + kLead) & (kRing - 1));
#endif
  };
  // The stage holding pair i + 2 is entered at the start of pair i's step (when pair
  // i + 2 is the first pair of its stage), so that the step can already read pair i + 2's
  // K. The slot refilled then held pair i, whose K and V every wave has read into
  // registers by then (the previous step read its V; lgkmcnt(0) before the barrier):
  // kLead <= kRing - 2. At that point the wave's only LDS reads in flight are pair
  // i + 1's K, which the step's first products need anyway.
  static_assert(kLead <= kRing - 2, "a refilled slot is no longer read");
  auto enter_mid = [&](int i) __attribute__((always_inline)) {
    const int j = i + 2;
    if (j % PPS == 0 && j / PPS < static_cast<int>(nst)) stage_enter(static_cast<uint32_t>(j / PPS));
  };
  auto pair_lds = [&](int i) __attribute__((always_inline)) {  // LDS byte address of pair i's K (its V is SB * 4 KiB on)
    return ring_base + ((static_cast<uint32_t>(i) / PPS) & (kRing - 1)) * (2 * SB * 256 * 16) +
           (static_cast<uint32_t>(i) % PPS) * 8192u;
  };
  auto read_k1 = [&](int i, half8 (&kk)[2][4], int r) {  // read r (h = r / 4, p = r % 4) of pair i's K
    const half8* kb = reinterpret_cast<const half8*>(
        reinterpret_cast<const char*>(&ring[0][0]) + (pair_lds(i) - ring_base));
    kk[r >> 2][r & 3] = kb[(r >> 2) * 256 + (r & 3) * 64 + lane];
  };
  auto read_k = [&](int i, half8 (&kk)[2][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 8; ++r) read_k1(i, kk, r);
  };
  // V^T operand of dim group j: row c is dim 16 j + c, element e is key
  // (e / 4) * 16 + 4 g + e % 4 of the pair (the order of P). Each half is one transposing
  // read: in a 16-lane group, lane i receives element i % 4 of the 8 bytes source lane
  // 4 e + i / 4 addressed, so source lane s (= c) addresses key 4 g + s / 4, dims
  // 16 j + 4 (s % 4) .. + 3, at its swizzled place.
  auto read_v1 = [&](int i, half8 (&va)[8], int j) {  // dim group j of pair i's V
    const uint32_t vb = pair_lds(i) + SB * 4096u;
    const lds_half4* p0 = reinterpret_cast<const lds_half4*>(
        reinterpret_cast<const __attribute__((address_space(3))) char*>(static_cast<uintptr_t>(vb)) + vtr_off[j]);
    const half4 lo = __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<lds_half4*>(p0)));
    const half4 hi = __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<lds_half4*>(p0 + 512)));
    va[j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  auto read_v = [&](int i, half8 (&va)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) read_v1(i, va, j);
  };
  // S^T of pair i for tile t: 2 accumulators (one per block); step k of 8 takes dims group
  // p = k % 4 of q's hi (k < 4) or lo part, so consecutive products into one accumulator
  // are 2 * NT MFMAs apart.
  auto qk_mfma = [&](const half8 (&kk)[2][4], floatx4 (&sc)[NT][2], int k, int t) __attribute__((always_inline)) {
    const int part = k >> 2, p = k & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      sc[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[h][p], part ? ql[t][p] : qh[t][p], sc[t][h], 0, 0, 0);
  };
  float x[NT][8];  // the current pair's masked x = s - m
  // Maxima of pair i (part one of its online softmax): masked x, and per lane the largest
  // of its 8. When some lane's exceeds its column's threshold (wave-uniform, rare after
  // a column's first keys), the column maxima move (`rescale`).
  auto maxima_tile = [&](auto masked, int i, const floatx4 (&sc)[NT][2], float (&x)[NT][8], float (&bm)[NT],
                         int t) __attribute__((always_inline)) {
    const int key0 = first_key + 32 * i;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        if constexpr (decltype(masked)::value) {
          const int kp = key0 + h * 16 + 4 * g + ii;
          // Bitwise, not short-circuit: straight-line selects instead of branches.
          const bool ok = (kp >= rlo[t]) & (kp <= rpos[t]) & (kp < key_end);
          x[t][h * 4 + ii] = ok ? sc[t][h][ii] : -INFINITY;
        } else {
          x[t][h * 4 + ii] = sc[t][h][ii];
        }
      }
    float b = kNoKey;
#pragma unroll
    for (int e = 0; e < 8; ++e) b = fmaxf(b, x[t][e]);
    bm[t] = b;
    pin(bm[t]);
  };
  auto maxima = [&](auto masked, int i, const floatx4 (&sc)[NT][2], float (&x)[NT][8], float (&bm)[NT]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < NT; ++t) maxima_tile(masked, i, sc, x, bm, t);
  };
  // The move: every column of the tile takes delta = max(0, its largest x) (a column's
  // first keys: their largest x, m being 0 until then), so that m becomes the running
  // maximum of its scores whenever some column's grew by more than kLazyRescale; the
  // accumulator and sum are scaled by 2^-delta (zero state for a first move) and the
  // pair's x shifted. A column still without a visible key keeps m = 0 and thr = kNoKey.
  auto rescale = [&](const float (&bm)[NT], float (&x)[NT][8]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (__builtin_amdgcn_ballot_w64(bm[t] > thr[t])) {  // wave-uniform
        const uint64_t a = PF_NOW();
        const float cm = max_xor32(max_xor16(bm[t]));
        const bool unset = thr[t] < 0.0f;
        const bool seen = cm > kNoKey;
        const float delta = unset ? (seen ? cm : 0.0f) : fmaxf(0.0f, cm);
        if (seen) thr[t] = kLazyRescale;
        const float corr = __builtin_amdgcn_exp2f(-delta);
        lsum[t] *= corr;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[t][j] *= corr;
        m[t] += delta;
        negm[t] = floatx4{-m[t], -m[t], -m[t], -m[t]};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[t][e] -= delta;
        pf_rare += PF_NOW() - a;
      }
    }
  };
  // Part two of pair i's softmax, in slices of 1-2 VALU each: P = 2^x (element e of a
  // lane is key (e / 4) * 16 + 4 g + e % 4 of the pair) as an f16 hi part and an f16 lo
  // part, and the sum. The lo part takes two mixed-precision fmas per element pair: lo =
  // f16(P - f32(hi)), a single rounding of the exact difference. Each slice pins its
  // inputs and outputs where it is called, so the compiler keeps it between the matrix
  // products it is meant to overlap (on gfx950 only about one VALU instruction per
  // 16x16x32 MFMA issues for free; every further one adds its own issue time).
  struct Soft {
    float pr[NT][8];
    half8 ph[NT], pl[NT];
    float rs[NT];
  };
  auto slice_exp = [&](Soft& sf, int t, int e) __attribute__((always_inline)) {
    pin(x[t][e]);
    sf.pr[t][e] = __builtin_amdgcn_exp2f(x[t][e]);
    pin(sf.pr[t][e]);
  };
  auto slice_hi = [&](Soft& sf, int t, int e) __attribute__((always_inline)) {
    const half2_t h2 = __builtin_convertvector(floatx2{sf.pr[t][2 * e], sf.pr[t][2 * e + 1]}, half2_t);
    sf.ph[t][2 * e] = h2[0];
    sf.ph[t][2 * e + 1] = h2[1];
    pin(sf.ph[t]);
  };
  auto slice_lo = [&](Soft& sf, int t, int e) __attribute__((always_inline)) {
    const uint32_t hp = __builtin_bit_cast(uint32_t, half2_t{sf.ph[t][2 * e], sf.ph[t][2 * e + 1]});
    uint32_t lp;
    __asm__ volatile(
        "v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, -1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=&v"(lp)
        : "v"(hp), "v"(sf.pr[t][2 * e]), "v"(sf.pr[t][2 * e + 1]));
    const half2_t l2 = __builtin_bit_cast(half2_t, lp);
    sf.pl[t][2 * e] = l2[0];
    sf.pl[t][2 * e + 1] = l2[1];
  };
  auto slice_sum = [&](Soft& sf, int t, int e) __attribute__((always_inline)) {
    pin(sf.pr[t][2 * e]);
    const float r2 = sf.pr[t][2 * e] + sf.pr[t][2 * e + 1];
    sf.rs[t] = e == 0 ? r2 : sf.rs[t] + r2;
    if (e == 3) lsum[t] += sf.rs[t];
    pin(sf.rs[t]);
  };
  // O^T += V^T P^T for tile t, dim group j (hi product; lo product with lo = true).
  auto pv_mfma = [&](const half8 (&va)[8], const Soft& sf, int t, int j, bool lo) __attribute__((always_inline)) {
    acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[j], lo ? sf.pl[t] : sf.ph[t], acc[t][j], 0, 0, 0);
  };
  auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

  // One pair step, software-pipelined one pair ahead in both LDS reads and scores. On
  // entry: pair i + 1's K is in kk, pair i's V in va, pair i's masked x (its rescale
  // done). Block one: pair i + 1's 16 * NT score MFMAs (starting from -m), with pair i's
  // exponentials and hi parts between them and pair i + 1's V reads (into vn). Halfway,
  // the next stage is entered. Block two: pair i's 8 * NT hi products with its lo parts
  // and pair i + 2's K reads (into kk) between them, then its 8 * NT lo products with its
  // sums and pair i + 1's maxima between them. Then pair i + 1's rescale, if some column's
  // maximum moved.
  half8 kk[2][4];
  auto step = [&](auto next_masked, int i, half8 (&va)[8], half8 (&vn)[8]) __attribute__((always_inline)) {
    PF_CYC(c0);
    enter_mid(i);
    PF_CYC(c1);
    __builtin_amdgcn_s_setprio(1);
    floatx4 scn[NT][2];
#pragma unroll
    for (int t = 0; t < NT; ++t) scn[t][0] = scn[t][1] = negm[t];
    Soft sf;
    constexpr int kMm = 16 * NT;  // score MFMAs
#pragma unroll
    for (int q = 0; q < kMm; ++q) {
      const int k = q / (2 * NT), t = (q / 2) % NT, h = q % 2;
      const int part = k >> 2, p = k & 3;
      scn[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[h][p], part ? ql[t][p] : qh[t][p], scn[t][h], 0, 0, 0);
      // 12 slices per tile over the 16 * NT products: the exponentials first, then
      // each hi pair once both of its exponentials are done.
#pragma unroll
      for (int sl = (q * 12 * NT) / kMm; sl < ((q + 1) * 12 * NT) / kMm; ++sl) {
        if (sl % 12 < 8) slice_exp(sf, sl / 12, sl % 12);
        else slice_hi(sf, sl / 12, sl % 12 - 8);
      }
      if (q % (kMm / 8) == kMm / 8 - 1) read_v1(i + 1, vn, q / (kMm / 8));
      fence();
    }
    float bmn[NT];
    PF_CYC(c2);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int t = 0; t < NT; ++t) pv_mfma(va, sf, t, j, false);
      // Unconditional (a pair past the wave's range reads ring data it never uses), so
      // the block stays one straight line of products and reads.
      read_k1(i + 2, kk, j);
#pragma unroll
      for (int sl = (j * 4 * NT) / 8; sl < ((j + 1) * 4 * NT) / 8; ++sl) slice_lo(sf, sl / 4, sl % 4);
      fence();
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) pin(sf.pl[t]);
    PF_CYC(c3);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int t = 0; t < NT; ++t) pv_mfma(va, sf, t, j, true);
#pragma unroll
      for (int sl = (j * 4 * NT) / 8; sl < ((j + 1) * 4 * NT) / 8; ++sl) slice_sum(sf, sl / 4, sl % 4);
      // The next pair's maxima, tile by tile, between the lo products.
      if (j % (8 / NT) == 8 / NT - 1) {
        const int t = j / (8 / NT);
        maxima_tile(next_masked, i + 1, scn, x, bmn, t);
      }
      fence();
    }
    PF_CYC(c4);
    __builtin_amdgcn_s_setprio(0);
    PF_ACC(pf_b0, c0, c1);
    PF_ACC(pf_b1, c1, c2);
    PF_ACC(pf_b2, c2, c3);
    PF_ACC(pf_b3, c3, c4);
#ifdef YX_PF_PROF
    pf_e1 += e1 - e0; pf_e2 += e2 - e1; pf_e3 += e3 - e2; pf_e4 += e4 - e3;
#endif
    rescale(bmn, x);
  };
  auto last = [&](int i, const half8 (&va)[8]) __attribute__((always_inline)) {
    Soft sf;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int e = 0; e < 8; ++e) slice_exp(sf, t, e);
#pragma unroll
      for (int e = 0; e < 4; ++e) slice_hi(sf, t, e);
#pragma unroll
      for (int e = 0; e < 4; ++e) slice_lo(sf, t, e);
#pragma unroll
      for (int e = 0; e < 4; ++e) slice_sum(sf, t, e);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int t = 0; t < NT; ++t) pv_mfma(va, sf, t, j, false);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int t = 0; t < NT; ++t) pv_mfma(va, sf, t, j, true);
    enter_mid(i);
  };

#ifdef YX_PF_PROF
  __builtin_amdgcn_sched_barrier(0);
  const uint64_t pf_rq = __builtin_amdgcn_s_memrealtime();
#endif
  stage_enter(0);  // pairs 0 .. PPS - 1
#ifdef YX_PF_PROF
  const uint64_t pf_rs = __builtin_amdgcn_s_memrealtime();
#endif
  const uint64_t pf_t1 = PF_NOW();
  (void)pf_t1;
  if (PPS == 1 && nst > 1) stage_enter(1);
  int i = 0;
  for (; i < pa; ++i) enter_mid(i);
  if (pa < pb) {
    half8 vaA[8], vaB[8];
    {  // The first pair's scores, maxima and V, and the next pair's K.
      read_k(pa, kk);
      floatx4 sc[NT][2];
#pragma unroll
      for (int t = 0; t < NT; ++t) sc[t][0] = sc[t][1] = floatx4{0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int t = 0; t < NT; ++t) qk_mfma(kk, sc, k, t);
      read_v(pa, vaA);
      if (pa + 1 < pb) read_k(pa + 1, kk);
      float bm[NT];
      if (pa >= wa && pa < wb)
        maxima(std::false_type{}, pa, sc, x, bm);
      else
        maxima(std::true_type{}, pa, sc, x, bm);
      rescale(bm, x);
    }
    // Steps by the kind of their next pair: masked before wa, whole in [wa, wb), masked
    // from wb. Two steps per turn, so that the V registers swap roles without copies.
    auto run = [&](auto next_masked, int i0, int end) __attribute__((always_inline)) {
      int ii = i0;
      for (; ii + 2 < end; ii += 2) {
        step(next_masked, ii, vaA, vaB);
        step(next_masked, ii + 1, vaB, vaA);
      }
      if (ii + 1 < end) {
        step(next_masked, ii, vaA, vaB);
#pragma unroll
        for (int j = 0; j < 8; ++j) vaA[j] = vaB[j];
        ++ii;
      }
      return ii;
    };
    i = run(std::true_type{}, i, min(wa, pb));
    i = run(std::false_type{}, i, wb);
    i = run(std::true_type{}, i, pb);
    last(i, vaA);
    ++i;
  }
  for (; i < npair; ++i) enter_mid(i);
  const uint64_t pf_t2 = PF_NOW();
  (void)pf_t2;
  PF_ADD(1, pf_t1 - pf_t0);
  PF_ADD(2, pf_t2 - pf_t1);
  PF_ADD(3, pf_stage);
  PF_ADD(4, pf_rare);
  PF_ADD(6, 1);
  PF_ADD(7, pb - pa);
  PF_ADD(8, pf_b0);
  PF_ADD(9, pf_b1);
  PF_ADD(10, pf_b2);
  PF_ADD(11, pf_b3);
#ifdef YX_PF_PROF
  (void)pf_e1; (void)pf_e2; (void)pf_e3; (void)pf_e4;
  PF_ADD(0, pf_rq);
  PF_ADD(3, pf_rs);
  PF_ADD(4, __builtin_amdgcn_s_memrealtime());
#endif
#ifdef YX_PF_PROF
  {
    uint32_t hw, xcc;
    __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    PF_ADD(12, pf_r0);
    PF_ADD(14, (static_cast<uint64_t>(xcc) << 32) | hw);
    PF_ADD(15, (static_cast<uint64_t>(blockIdx.x) << 32) | static_cast<uint32_t>(npair));
  }
#endif
  // No load into LDS may land after the workgroup ends.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const size_t qd = static_cast<size_t>(hq) * kD;
  const uint32_t nch = it.chunk_nch >> 16;
  if (nch <= 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float l = sum_xor32(sum_xor16(lsum[t]));
      const uint32_t lr = (wave * NT + t) * 16 + c;
      if (lr >= nlog) continue;
      const uint32_t rr = it.r0 + lr / G, h = kh * G + lr % G;
      // acc[t][j][i] is dim 16 j + 4 g + i of the column.
      float* o = out + rr * qd + h * kD + g * 4;
      const float inv = 1.0f / l;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        *reinterpret_cast<float4*>(o + j * 16) =
            float4{acc[t][j][0] * inv, acc[t][j][1] * inv, acc[t][j][2] * inv, acc[t][j][3] * inv};
    }
    (void)pf_t2;
#ifdef YX_PF_PROF
    PF_ADD(5, __builtin_amdgcn_s_memrealtime());
    __builtin_amdgcn_s_waitcnt(0);
    PF_ADD(13, __builtin_amdgcn_s_memrealtime());
#endif
    return;
  }
  // A split tile: this chunk's (maximum, sum, unnormalised O) of each column go to its
  // partial slot (`[slot][kv head][kPrefillRows][128]`, device-coherent stores), and the
  // tile's last chunk to arrive merges the chunks in chunk order (the split-K hand-off
  // of the decode kernels, with the same memory-order argument; merge_tile).
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(part_o, part_o_bytes);
  const __amdgpu_buffer_rsrc_t rml = make_rsrc(part_ml, part_ml_bytes);
  const size_t slot = (static_cast<size_t>(it.part_base) + (it.chunk_nch & 0xffffu)) * hkv + kh;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float l = sum_xor32(sum_xor16(lsum[t]));
    const uint32_t lr = (wave * NT + t) * 16 + c;
    if (lr >= nlog) continue;
    const size_t e = slot * kPrefillRows + lr;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      st4_coherent(ro, static_cast<uint32_t>((e * kD + 16 * j + 4 * g) * 4),
                   float4{acc[t][j][0], acc[t][j][1], acc[t][j][2], acc[t][j][3]});
    if (g == 0) st2_coherent(rml, static_cast<uint32_t>(e * 8), float2{m[t], l});
  }
  __builtin_amdgcn_s_waitcnt(0);
  __shared__ uint32_t last_chunk;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* cnt = counters + (static_cast<size_t>(it.counter) * hkv + kh) * kCounterStride;
    const uint32_t arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_chunk = arrived == nch - 1;
    if (last_chunk) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last_chunk) return;
  merge_tile<64 * W, kPrefillRows>(it.r0, it.nrows, it.part_base, nch, kh, G, hq, hkv, out, ro, rml);
}

}  // namespace yx
