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

#include "attn_decode.hpp"

namespace yx {

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
  // the arena, [p][g][key] in LDS): lane l fetches key l % 16, dims group l / 16.
  static_assert(kPrefillWaves == 8 && SB == 4, "the stage split below assumes 8 waves, 4 blocks");
  constexpr int kRowsPerWave = 4;  // 1 KiB rows (loads) per wave per stage
  const uint32_t my_blk = static_cast<uint32_t>(wave >> 1);
  const bool my_v = (wave & 1) != 0;
  const uint32_t my_row0 = 0;
  const uint32_t lane_src = my_v ? static_cast<uint32_t>(lane) * 16u
                                 : static_cast<uint32_t>((lane & 15) * 4 + (lane >> 4)) * 16u;
  const char* my_arena = reinterpret_cast<const char*>(my_v ? vc : kc);
  const uint32_t ring_base = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) half8*)&ring[0][0]));
  auto issue = [&](uint32_t st, uint32_t slot) {  // stage st into ring slot `slot`
    uint32_t b = it.blk0 + st * SB + my_blk;
    b = b < it.blk1 ? b : it.blk1 - 1;  // past the end: re-read the last block (unused)
    const uint32_t page = pt[b >> bpp_shift];
    const char* blk = my_arena + ((static_cast<size_t>(page) * hkv + kh) * head_stride +
                                  static_cast<size_t>(b & bpp_mask) * 16 * kD) * 2;
    const uint32_t dst = ring_base + slot * (2 * SB * 256 * 16) +
                         (my_v ? SB * 4096u : 0u) + my_blk * 4096u;
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
      load_to_lds16(blk + (my_row0 + r) * 1024 + lane_src, dst + (my_row0 + r) * 1024);
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

  float m[NT], l[NT];
  floatx4 acc[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m[t] = -INFINITY;
    l[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[t][j] = floatx4{0, 0, 0, 0};
  }
  const int key_end = static_cast<int>(it.blk1 * 16);

  auto compute = [&](const half8* kbuf, const half8* vbuf, uint32_t s0) {
    // Two blocks (32 keys) per softmax update; PV as 16x16x32 products over both.
#pragma unroll
    for (int pr2 = 0; pr2 < SB / 2; ++pr2) {
      const int key0 = static_cast<int>((s0 + 2 * pr2) * 16);
      if (key0 > wmax || key0 + 31 < wlo || key0 >= key_end) continue;  // uniform
      half8 kk[2][4], vv[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int base = (2 * pr2 + h) * 256;
#pragma unroll
        for (int p = 0; p < 4; ++p) kk[h][p] = kbuf[base + p * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) vv[h][i] = vbuf[base + (4 * g + i) * 16 + c];
      }
      // Scores of every (tile, block): 2 * NT accumulators, each taking the hi-part
      // products for p = 0..3 and then the lo-part ones, so consecutive products into one
      // accumulator are 2 * NT MFMAs apart and no add joins the parts afterwards.
      floatx4 sc[NT][2];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) sc[t][h] = floatx4{0, 0, 0, 0};
#pragma unroll
      for (int part = 0; part < 2; ++part)
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h)
              sc[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[h][p], part ? ql[t][p] : qh[t][p],
                                                                sc[t][h], 0, 0, 0);
      half8 ph[NT], pl[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        // Every key of the pair visible to every row of the tile: no mask needed.
        const bool whole = (key0 + 31 <= tmin[t]) & (key0 >= tlo[t]) & (key0 + 32 <= key_end);
        float x[8], bmax = -INFINITY;
        if (whole) {  // uniform: the common case needs no mask
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              x[h * 4 + i] = sc[t][h][i];
              bmax = fmaxf(bmax, x[h * 4 + i]);
            }
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int kp = key0 + h * 16 + 4 * g + i;
              // Bitwise, not short-circuit: straight-line selects instead of branches.
              const bool ok = (kp >= rlo[t]) & (kp <= rpos[t]) & (kp < key_end);
              x[h * 4 + i] = ok ? sc[t][h][i] : -INFINITY;
              bmax = fmaxf(bmax, x[h * 4 + i]);
            }
        }
        bmax = max_xor32(max_xor16(bmax));
        // The running maximum moves only when some column's maximum grew by more than
        // kLazyRescale (or was still empty): between moves, scores may exceed it by up
        // to that, so P stays below 2^kLazyRescale, well inside binary16 and f32. The
        // result is the same softmax (the sum uses the same offset); most stages then
        // skip the rescale of the accumulators.
        const float mn = fmaxf(m[t], bmax);
        if (__builtin_amdgcn_ballot_w64(mn > m[t] + kLazyRescale)) {  // wave-uniform
          const float corr = mn != -INFINITY ? __builtin_amdgcn_exp2f(m[t] - mn) : 1.0f;
          l[t] *= corr;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[t][j] *= corr;
          m[t] = mn;
        }
        // A whole tile has a finite maximum by now; otherwise a column that has seen no
        // key yet (maximum -inf) gets zeros.
        const bool live = whole || m[t] != -INFINITY;
        float pr[8], rs = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pr[i] = live ? __builtin_amdgcn_exp2f(x[i] - m[t]) : 0.0f;
          rs += pr[i];
        }
        rs = sum_xor32(sum_xor16(rs));
        l[t] += rs;
        // P as an f16 hi part plus an f16 lo part; element e of a lane is key
        // (e / 4) * 16 + 4g + e % 4 of the pair, as the V operand below.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ph[t][e] = static_cast<_Float16>(pr[e]);
          if constexpr (kPrefillSplitP) pl[t][e] = static_cast<_Float16>(pr[e] - static_cast<float>(ph[t][e]));
        }
      }
      // PV: every (tile, dim group) hi product, then every lo product, so that the
      // two products into one accumulator are 8 * NT MFMAs apart.
      half8 va[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        va[j] = half8{vv[0][0][j], vv[0][1][j], vv[0][2][j], vv[0][3][j],
                      vv[1][0][j], vv[1][1][j], vv[1][2][j], vv[1][3][j]};
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[j], ph[t], acc[t][j], 0, 0, 0);
      if constexpr (kPrefillSplitP) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[j], pl[t], acc[t][j], 0, 0, 0);
      }
    }
  };

  uint32_t slot = 0;
  for (uint32_t st = 0; st < nst; ++st) {
    // This wave's loads of stage st are done when at most the kRing - 2 later stages'
    // (kRowsPerWave loads each) are in flight; the barrier then makes every wave's part visible,
    // and every wave has finished the stage before (whose slot is refilled next).
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(kRowsPerWave * (kRing - 2)) : "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    issue(st + kRing - 1, slot == 0 ? kRing - 1 : slot - 1);
    compute(&ring[slot][0], &ring[slot][SB * 256], it.blk0 + st * SB);
    slot = slot + 1 == kRing ? 0 : slot + 1;
  }
  // No load into LDS may land after the workgroup ends.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const size_t qd = static_cast<size_t>(hq) * kD;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint32_t lr = (wave * NT + t) * 16 + c;
    if (lr >= nlog) continue;
    const uint32_t rr = it.r0 + lr / G, h = kh * G + lr % G;
    float* o = out + rr * qd + h * kD + g * 32;
    const float inv = 1.0f / l[t];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<float4*>(o + i * 8) =
          float4{acc[t][0][i] * inv, acc[t][1][i] * inv, acc[t][2][i] * inv, acc[t][3][i] * inv};
      *reinterpret_cast<float4*>(o + i * 8 + 4) =
          float4{acc[t][4][i] * inv, acc[t][5][i] * inv, acc[t][6][i] * inv, acc[t][7][i] * inv};
    }
  }
}

}  // namespace yx
