// Paged prefill / chunked-prefill attention for gfx950: MFMA tiles over K/V staged in LDS.
//
// The same arithmetic as `LayerPass::attend` (crates/yaxus-backend-cpu/src/lib.rs:
// 389-427) for passes with many rows per sequence, the shape the reference's tiled
// kernel serves (ATTN_TILE, crates/yaxus-backend-gpu/src/shaders.rs:422-592: 32 rows x
// 32-key blocks, f32 SIMT). Here a workgroup of 8 waves (two per SIMD) takes a tile of
// kPrefillRows logical rows, the (row, query head) pairs of consecutive rows of one
// sequence and one KV head; each wave owns 16 of them, the 16 columns of its MFMA tile.
// Keys stream from HBM straight into a 4-stage LDS ring of 64-key stages
// (global_load_lds_dwordx4, no registers; three stages in flight while one is computed),
// and every wave reads them there. Per 32 keys:
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
// (causal, window) are skipped by that wave.
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
  uint32_t blk0;    // first key block any row of the tile can see
  uint32_t blk1;    // one past the last key block any row of the tile can see
  uint32_t pad[3];
};

static constexpr int kPrefillWaves = 8;
static constexpr int kPrefillTiles = 1;  // MFMA tiles (16 logical rows) per wave
static constexpr int kPrefillRows = kPrefillWaves * kPrefillTiles * 16;  // logical rows per item

static constexpr int kStageBlocks = 4;  // 16-key blocks per LDS stage (64 keys, 32 KiB of K+V)
static constexpr int kRing = 4;         // LDS stages: kRing - 1 in flight while one is computed
static constexpr bool kPrefillSplitP = true;  // P as f16 hi + lo (else one f16 rounding)
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

// Two waves per SIMD (at most 256 registers each), so one wave's softmax arithmetic
// overlaps the other's matrix products.
// QKV: q is not given; the kernel reads its rows' raw q heads from qkv and normalises
// and rotates them itself, with write_rows' arithmetic (the same bits as
// qk_norm_rope_append), the key heads having been stored before the launch.
template <bool QKV>
__global__ __launch_bounds__(64 * kPrefillWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void paged_attn_prefill(
    const PrefillItem* __restrict__ items, const uint32_t* pos,
    const uint32_t* __restrict__ pages, const _Float16* __restrict__ kc,
    const _Float16* __restrict__ vc, const float* q, float* __restrict__ out,
    uint32_t hq, uint32_t hkv, uint32_t bpp_shift, uint32_t window, float scale_log2,
    QkvIn qi_in) {
  constexpr int NT = kPrefillTiles, SB = kStageBlocks;
  // A ring of stages; each holds SB blocks of K as [p][g][key] (4 KiB each) and then SB
  // blocks of V as [key][128] (4 KiB each).
  __shared__ half8 ring[kRing][2 * SB * 256];
  // One dimension, KV head fastest: workgroups start in the host's longest-first item
  // order across all KV heads.
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
  // Each wave moves an eighth of a stage: wave w takes block w / 2 of the stage, its K
  // (w even) or V (w odd), as four 1 KiB rows. K row p is read transposed ([p][key][g] in
  // the arena, [p][g][key] in LDS): lane l fetches key l % 16, dims group l / 16. V keeps
  // its [key][128] rows, but the 32-byte chunks of key k's row are stored XOR-swizzled
  // (chunk j at j ^ (k & 7)) so that the transposing reads below stay at the minimum of
  // two passes per 512 bytes; within a 1 KiB row lane l lands on key 4r + l / 16, piece
  // l % 16, and so fetches the piece that belongs there.
  static_assert(kPrefillWaves == 8 && SB == 4, "the stage split below assumes 8 waves, 4 blocks");
  constexpr int kRowsPerWave = 4;  // 1 KiB rows (loads) per wave per stage
  const uint32_t my_blk = static_cast<uint32_t>(wave >> 1);
  const bool my_v = (wave & 1) != 0;
  uint32_t lane_src[kRowsPerWave];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) {
    const uint32_t key = 4 * r + (lane >> 4), pp = lane & 15;
    lane_src[r] = my_v ? key * 256u + (2u * ((pp >> 1) ^ (key & 7u)) + (pp & 1u)) * 16u
                       : static_cast<uint32_t>(r * 1024 + ((lane & 15) * 4 + (lane >> 4)) * 16);
  }
  const char* my_arena = reinterpret_cast<const char*>(my_v ? vc : kc);
  const uint32_t ring_base = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) half8*)&ring[0][0]));
  // The page of the block a wave moves for stage st is read one stage ahead, so the
  // scalar load's latency is not waited for right after the stage's barrier.
  auto page_of = [&](uint32_t st) {
    uint32_t b = it.blk0 + st * SB + my_blk;
    b = b < it.blk1 ? b : it.blk1 - 1;  // past the end: re-read the last block (unused)
    return pt[b >> bpp_shift] * hkv * head_stride + static_cast<size_t>(b & bpp_mask) * 16 * kD;
  };
  size_t next_elem = page_of(0);
  auto issue = [&](uint32_t st, uint32_t slot) {  // stage st into ring slot `slot`
    const char* blk = my_arena + (next_elem + kh * head_stride) * 2;
    next_elem = page_of(st + 1);
    const uint32_t dst = ring_base + slot * (2 * SB * 256 * 16) +
                         (my_v ? SB * 4096u : 0u) + my_blk * 4096u;
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) load_to_lds16(blk + lane_src[r], dst + r * 1024);
  };
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
#pragma unroll
  for (int j = 0; j < kRing - 1; ++j) issue(j, j);

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

  static_assert(NT == 1, "the pipelined loop below takes one MFMA tile per wave");
  float m = -INFINITY;
  float lsum = 0.0f;  // this lane's share of its column's sum (its 8 keys of every pair)
  floatx4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = floatx4{0, 0, 0, 0};
  const int key_end = static_cast<int>(it.blk1 * 16);
  const int first_key = static_cast<int>(it.blk0 * 16);
  const int npair = static_cast<int>(2 * nst);
  // Pair i holds keys first_key + 32 i .. + 31. This wave computes the pairs [pa, pb) that
  // hold a key some column of the wave can see; the others it only passes through.
  int pa = npair, pb = npair;
  if (wmax >= 0) {
    const int d = wlo - first_key;
    pa = d <= 0 ? 0 : d / 32;
    const int e = min(wmax, key_end - 1) - first_key;
    pb = e < 0 ? 0 : min(npair, e / 32 + 1);
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
  // kRing - 2 later stages' are in flight, and the barrier makes every wave's part
  // visible. Every wave has then also issued and (lgkmcnt) finished its reads of the
  // stage before st, whose slot is refilled with stage st + kRing - 1.
  auto stage_enter = [&](uint32_t st) {
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)" ::"n"(kRowsPerWave * (kRing - 2))
                     : "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    issue(st + kRing - 1, (st + kRing - 1) & (kRing - 1));
  };
  auto pair_lds = [&](int i) {  // LDS byte address of pair i's K (its V is 16 KiB on)
    return ring_base + ((static_cast<uint32_t>(i) >> 1) & (kRing - 1)) * (2 * SB * 256 * 16) +
           (static_cast<uint32_t>(i) & 1u) * 8192u;
  };
  // S^T of pair i: 2 accumulators (one per block), each taking the hi-part products for
  // p = 0..3 and then the lo-part ones, 2 MFMAs apart.
  auto qk = [&](int i, floatx4 (&sc)[2]) {
    const half8* kb = reinterpret_cast<const half8*>(
        reinterpret_cast<const char*>(&ring[0][0]) + (pair_lds(i) - ring_base));
    half8 kk[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int p = 0; p < 4; ++p) kk[h][p] = kb[h * 256 + p * 64 + lane];
#pragma unroll
    for (int h = 0; h < 2; ++h) sc[h] = floatx4{0, 0, 0, 0};
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[h][p], part ? ql[0][p] : qh[0][p], sc[h], 0, 0, 0);
  };
  // V^T operand of dim group j: row c is dim 16 j + c, element e is key
  // (e / 4) * 16 + 4 g + e % 4 of the pair (the order of P). Each half is one transposing
  // read: in a 16-lane group, lane i receives element i % 4 of the 8 bytes source lane
  // 4 e + i / 4 addressed, so source lane s (= c) addresses key 4 g + s / 4, dims
  // 16 j + 4 (s % 4) .. + 3, at its swizzled place.
  auto read_v = [&](int i, half8 (&va)[8]) {
    const uint32_t vb = pair_lds(i) + SB * 4096u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const lds_half4* p0 = reinterpret_cast<const lds_half4*>(
          reinterpret_cast<const __attribute__((address_space(3))) char*>(static_cast<uintptr_t>(vb)) + vtr_off[j]);
      const half4 lo = __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<lds_half4*>(p0)));
      const half4 hi = __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<lds_half4*>(p0 + 512)));
      va[j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };
  // Online softmax of pair i for the wave's columns, in two parts. The running maximum
  // moves only when some column's maximum grew by more than kLazyRescale (or was still
  // empty): between moves, scores may exceed it by up to that, so P stays below
  // 2^kLazyRescale, well inside binary16 and f32; the sum uses the same offset, so the
  // softmax is the same. Part one masks the scores, finds the maxima and, when the
  // maximum moves (wave-uniform, rare after the first pairs), rescales the accumulators
  // and the sum in place.
  auto rescale = [&](auto masked, int i, const floatx4 (&sc)[2], float (&x)[8]) {
    const int key0 = first_key + 32 * i;
    float bmax = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        if constexpr (decltype(masked)::value) {
          const int kp = key0 + h * 16 + 4 * g + ii;
          // Bitwise, not short-circuit: straight-line selects instead of branches.
          const bool ok = (kp >= rlo[0]) & (kp <= rpos[0]) & (kp < key_end);
          x[h * 4 + ii] = ok ? sc[h][ii] : -INFINITY;
        } else {
          x[h * 4 + ii] = sc[h][ii];
        }
        bmax = fmaxf(bmax, x[h * 4 + ii]);
      }
    bmax = max_xor32(max_xor16(bmax));
    const float mn = fmaxf(m, bmax);
    if (__builtin_amdgcn_ballot_w64(mn > m + kLazyRescale)) {  // wave-uniform
      // A column still empty after this pair (mn = -inf) keeps its (zero) state.
      const float corr = mn != -INFINITY ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
      lsum *= corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= corr;
      m = mn;
    }
  };
  // Part two: P as f16 hi + lo parts (element e of a lane is key (e / 4) * 16 + 4 g + e % 4
  // of the pair) and this lane's share of the sum. Unmasked pairs are whole for every
  // column, so m is finite there; a masked column that has seen no key yet (m = -inf)
  // gets zeros.
  auto probs = [&](auto masked, const float (&x)[8], half8& ph, half8& pl) {
    float pr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (decltype(masked)::value)
        pr[e] = m != -INFINITY ? __builtin_amdgcn_exp2f(x[e] - m) : 0.0f;
      else
        pr[e] = __builtin_amdgcn_exp2f(x[e] - m);
    }
    float rs = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) rs += pr[e];
    lsum += rs;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ph[e] = static_cast<_Float16>(pr[e]);
      if constexpr (kPrefillSplitP) pl[e] = static_cast<_Float16>(pr[e] - static_cast<float>(ph[e]));
    }
  };
  // O^T += V^T P^T: every dim group's hi product, then every lo product (the two products
  // into one accumulator 8 MFMAs apart).
  auto pv = [&](const half8 (&va)[8], const half8& ph, const half8& pl) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[j], ph, acc[j], 0, 0, 0);
    if constexpr (kPrefillSplitP) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[j], pl, acc[j], 0, 0, 0);
    }
  };
  // One pair step, software-pipelined: this pair's V is read (LDS) while its maxima are
  // found; the next pair's scores (16 MFMAs) are interleaved with this pair's
  // exponentials (VALU) in one block; then this pair's products. The scores of pair i
  // arrive in sc, and pair i + 1's leave in it. At the end of a stage (odd i) the next
  // stage is entered between this pair's reads and the next pair's.
  floatx4 sc[2];
  auto step = [&](auto masked, auto has_next, int i) {
    half8 va[8];
    read_v(i, va);
    float x[8];
    rescale(masked, i, sc, x);
    if ((i & 1) && (i >> 1) + 1 < static_cast<int>(nst)) stage_enter(static_cast<uint32_t>(i >> 1) + 1);
    half8 ph, pl;
    if constexpr (decltype(has_next)::value) {
      // The next pair's K, then its 16 score MFMAs two at a time (one per block, so two
      // independent chains), each couple followed by a slice of this pair's softmax. The
      // sched_barrier fences keep this order: the matrix pipe runs the products while
      // the vector pipe does the slices.
      const half8* kb = reinterpret_cast<const half8*>(
          reinterpret_cast<const char*>(&ring[0][0]) + (pair_lds(i + 1) - ring_base));
      half8 kk[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int p = 0; p < 4; ++p) kk[h][p] = kb[h * 256 + p * 64 + lane];
      floatx4 scn[2] = {floatx4{0, 0, 0, 0}, floatx4{0, 0, 0, 0}};
      float pr[8], rs = 0.0f;
      floatx2 hf[4];  // ph as f32, pairwise
      auto mm = [&](int k) {  // score MFMAs k (hi parts p = k, then lo parts p = k - 4)
        const int p = k & 3;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          scn[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[h][p], k < 4 ? qh[0][p] : ql[0][p], scn[h], 0, 0, 0);
      };
      auto ex = [&](int e) {
        if constexpr (decltype(masked)::value)
          pr[e] = m != -INFINITY ? __builtin_amdgcn_exp2f(x[e] - m) : 0.0f;
        else
          pr[e] = __builtin_amdgcn_exp2f(x[e] - m);
      };
      auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
      ex(0); ex(1); ex(2); ex(3);
      fence();
      mm(0); ex(4); ex(5); ex(6); ex(7);
      fence();
      mm(1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const half2_t h2 = __builtin_convertvector(floatx2{pr[2 * e], pr[2 * e + 1]}, half2_t);
        ph[2 * e] = h2[0];
        ph[2 * e + 1] = h2[1];
      }
      fence();
      mm(2);
#pragma unroll
      for (int e = 0; e < 4; ++e) hf[e] = __builtin_convertvector(half2_t{ph[2 * e], ph[2 * e + 1]}, floatx2);
      fence();
      mm(3);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const floatx2 d = floatx2{pr[2 * e], pr[2 * e + 1]} - hf[e];
        const half2_t l2 = __builtin_convertvector(d, half2_t);
        pl[2 * e] = l2[0];
        pl[2 * e + 1] = l2[1];
      }
      fence();
      mm(4);
#pragma unroll
      for (int e = 0; e < 8; ++e) rs += pr[e];
      fence();
      mm(5);
      lsum += rs;
      fence();
      mm(6);
      fence();
      mm(7);
      fence();
      pv(va, ph, pl);
      sc[0] = scn[0];
      sc[1] = scn[1];
    } else {
      probs(masked, x, ph, pl);
      pv(va, ph, pl);
    }
  };
  // The wave's pairs in three runs: those needing the mask (before the window has
  // passed every column's start), those every column sees whole, and masked ones again
  // (the causal diagonal and the end of the keys). Pairs outside [pa, pb) only enter
  // their stages.
  int wa = pa, wb = pa;
  if (pa < pb) {
    const int d = tlo[0] - first_key;
    wa = d <= 0 ? 0 : (d + 31) / 32;
    const int e = min(tmin[0] - 31, key_end - 32) - first_key;
    wb = e < 0 ? 0 : e / 32 + 1;
    wa = min(max(wa, pa), pb - 1);
    wb = min(max(wb, wa), pb - 1);
  }
  stage_enter(0);
  int i = 0;
  for (; i < pa; ++i)
    if ((i & 1) && (i >> 1) + 1 < static_cast<int>(nst)) stage_enter(static_cast<uint32_t>(i >> 1) + 1);
  if (pa < pb) {
    qk(pa, sc);
    for (; i < wa; ++i) step(std::true_type{}, std::true_type{}, i);
    for (; i < wb; ++i) step(std::false_type{}, std::true_type{}, i);
    for (; i < pb - 1; ++i) step(std::true_type{}, std::true_type{}, i);
    step(std::true_type{}, std::false_type{}, i);
    ++i;
  }
  for (; i < npair; ++i)
    if ((i & 1) && (i >> 1) + 1 < static_cast<int>(nst)) stage_enter(static_cast<uint32_t>(i >> 1) + 1);
  // No load into LDS may land after the workgroup ends.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const float l = sum_xor32(sum_xor16(lsum));
  const size_t qd = static_cast<size_t>(hq) * kD;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint32_t lr = (wave * NT + t) * 16 + c;
    if (lr >= nlog) continue;
    const uint32_t rr = it.r0 + lr / G, h = kh * G + lr % G;
    // acc[t][j][i] is dim 16 j + 4 g + i of the column.
    float* o = out + rr * qd + h * kD + g * 4;
    const float inv = 1.0f / l;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<float4*>(o + j * 16) =
          float4{acc[j][0] * inv, acc[j][1] * inv, acc[j][2] * inv, acc[j][3] * inv};
  }
}

}  // namespace yx
