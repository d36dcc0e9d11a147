// Paged prefill / chunked-prefill attention for gfx950: MFMA tiles over K/V staged in LDS.
//
// The same arithmetic as `LayerPass::attend` (crates/yaxus-backend-cpu/src/lib.rs:
// 389-427) for passes with many rows per sequence, the shape the reference's tiled
// kernel serves (ATTN_TILE, crates/yaxus-backend-gpu/src/shaders.rs:422-592: 32 rows x
// 32-key blocks, f32 SIMT). Here a workgroup of 4 waves takes a tile of consecutive
// rows of one sequence and one KV head; its (row, query head) pairs are logical rows,
// 32 per wave as 2 MFMA tiles of 16 columns. Keys stream through LDS in stages of 2
// blocks of 16 (two buffers: stage s+1 is fetched from HBM into registers while stage s
// is computed, then written to the other buffer), and every wave reads them there:
//   S^T[key][row] = K . Q^T      8 x v_mfma_f32_16x16x32_f16 per tile (q as hi + lo f16)
//   online softmax per column, once per 32 keys (xor-16 swizzle, 32-lane shuffle);
//   the accumulator is rescaled only when a column's maximum moved
//   O^T += V^T P^T               16 x v_mfma_f32_16x16x32_f16 per tile and 32 keys (P hi + lo)
// q and P each go in as a binary16 hi part plus a lo part, two products into one
// result, so both keep ~2^-22 relative accuracy (a single rounding costs up to 6e-4
// absolute on few-key rows); K and V are binary16 already. This doubles the MFMA work
// of the plain-f16 form. The tests compare with the f32 oracle and an f64 brute force.
// Blocks no row of a wave can see (causal, window) are skipped by that wave.
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

static constexpr int kPrefillWaves = 4;
static constexpr int kPrefillTiles = 2;  // MFMA tiles (16 logical rows) per wave
static constexpr int kPrefillRows = kPrefillWaves * kPrefillTiles * 16;  // logical rows per item

static constexpr int kStageBlocks = 2;  // 16-key blocks per LDS stage (32 keys, 16 KiB of K+V)

__global__ __launch_bounds__(64 * kPrefillWaves) void paged_attn_prefill(
    const PrefillItem* __restrict__ items, const uint32_t* __restrict__ pos,
    const uint32_t* __restrict__ pages, const _Float16* __restrict__ kc,
    const _Float16* __restrict__ vc, const float* __restrict__ q, float* __restrict__ out,
    uint32_t hq, uint32_t hkv, uint32_t bpp_shift, uint32_t window, float scale_log2) {
  constexpr int NT = kPrefillTiles, SB = kStageBlocks;
  __shared__ half8 kbuf[2][SB * 256];  // a stage of K blocks (4 KiB each), [p][g][key]
  __shared__ half8 vbuf[2][SB * 256];  // and of V
  const PrefillItem it = items[blockIdx.x];
  const uint32_t kh = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, g = lane >> 4;
  const uint32_t G = hq / hkv;
  const uint32_t nlog = it.nrows * G;

  const uint32_t bpp_mask = (1u << bpp_shift) - 1u;
  const size_t head_stride = static_cast<size_t>(16u << bpp_shift) * kD;
  const uint32_t* pt = pages + it.pt_off;
  auto block_ptr = [&](uint32_t b, const _Float16* base) {
    b = b < it.blk1 ? b : it.blk1 - 1;  // past the end: re-read the last block (masked)
    const uint32_t page = pt[b >> bpp_shift];
    return reinterpret_cast<const half8*>(base + (static_cast<size_t>(page) * hkv + kh) * head_stride +
                                          static_cast<size_t>(b & bpp_mask) * 16 * kD);
  };
  half8 kreg[SB], vreg[SB];
  auto fetch = [&](uint32_t b0) {
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      kreg[i] = __builtin_nontemporal_load(block_ptr(b0 + i, kc) + tid);
      vreg[i] = __builtin_nontemporal_load(block_ptr(b0 + i, vc) + tid);
    }
  };
  fetch(it.blk0);  // the first stage is in flight while q is set up

  half8 qh[NT][4], ql[NT][4];  // q as binary16 hi + lo parts
  int rpos[NT], rlo[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint32_t lr = (wave * NT + t) * 16 + c;
    rpos[t] = -1;
    rlo[t] = 0;
    if (lr < nlog) {
      const uint32_t rr = it.r0 + lr / G, h = kh * G + lr % G;
      const int p = static_cast<int>(pos[rr]);
      rpos[t] = p;
      rlo[t] = (window > 0 && p + 1 > static_cast<int>(window)) ? p + 1 - static_cast<int>(window) : 0;
      const float* qp = q + (static_cast<size_t>(rr) * hq + h) * kD + g * 8;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const float4 a = *reinterpret_cast<const float4*>(qp + pp * 32);
        const float4 b = *reinterpret_cast<const float4*>(qp + pp * 32 + 4);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qh[t][pp][e] = static_cast<_Float16>(x[e]);
          ql[t][pp][e] = static_cast<_Float16>(x[e] - static_cast<float>(qh[t][pp][e]));
        }
      }
    } else {
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) qh[t][pp] = ql[t][pp] = half8{0, 0, 0, 0, 0, 0, 0, 0};
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

  for (uint32_t s0 = it.blk0; s0 < it.blk1; s0 += SB) {
    const int buf = ((s0 - it.blk0) / SB) & 1;
    // K goes to LDS as [p][g][key] (the arena's [p][key][g] transposed within each 1 KiB
    // row group), so that each wave's operand reads are 64 consecutive 16-byte pieces.
    const int kdst = (tid & ~63) | ((tid & 3) << 4) | ((tid >> 2) & 15);
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      kbuf[buf][i * 256 + kdst] = kreg[i];
      vbuf[buf][i * 256 + tid] = vreg[i];
    }
    __syncthreads();
    if (s0 + SB < it.blk1) fetch(s0 + SB);  // the next stage streams in during this one
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
        for (int p = 0; p < 4; ++p) kk[h][p] = kbuf[buf][base + p * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) vv[h][i] = vbuf[buf][base + (4 * g + i) * 16 + c];
      }
      // Scores of every (tile, block) with p outermost: 4 * NT independent MFMA chains
      // of 4 each (hi and lo parts of q), so the MFMA latency is hidden by the others.
      floatx4 sh[NT][2], sl[NT][2];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) sh[t][h] = sl[t][h] = floatx4{0, 0, 0, 0};
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            sh[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[h][p], qh[t][p], sh[t][h], 0, 0, 0);
            sl[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk[h][p], ql[t][p], sl[t][h], 0, 0, 0);
          }
      floatx4 sc[NT][2];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) sc[t][h] = sh[t][h] + sl[t][h];
      half8 ph[NT], pl[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        // Every key of the pair visible to every row of the tile: no mask needed.
        const bool whole = (key0 + 31 <= tmin[t]) & (key0 >= tlo[t]) & (key0 + 32 <= key_end);
        float x[8], bmax = -INFINITY;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kp = key0 + h * 16 + 4 * g + i;
            const float v = sc[t][h][i] * scale_log2;
            // Bitwise, not short-circuit: straight-line selects instead of branches.
            const bool ok = whole | ((kp >= rlo[t]) & (kp <= rpos[t]) & (kp < key_end));
            x[h * 4 + i] = ok ? v : -INFINITY;
            bmax = fmaxf(bmax, x[h * 4 + i]);
          }
        bmax = fmaxf(bmax, xor16(bmax));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float mn = fmaxf(m[t], bmax);
        const bool live = mn != -INFINITY;
        float pr[8], rs = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pr[i] = live ? __builtin_amdgcn_exp2f(x[i] - mn) : 0.0f;
          rs += pr[i];
        }
        rs += xor16(rs);
        rs += __shfl_xor(rs, 32);
        // Rescale only when some column's maximum moved (wave-uniform test).
        if (__builtin_amdgcn_ballot_w64(mn != m[t])) {
          const float corr = live ? __builtin_amdgcn_exp2f(m[t] - mn) : 1.0f;
          l[t] *= corr;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[t][j] *= corr;
        }
        l[t] += rs;
        m[t] = mn;
        // P as an f16 hi part plus an f16 lo part; element e of a lane is key
        // (e / 4) * 16 + 4g + e % 4 of the pair, as the V operand below.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ph[t][e] = static_cast<_Float16>(pr[e]);
          pl[t][e] = static_cast<_Float16>(pr[e] - static_cast<float>(ph[t][e]));
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
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[j], pl[t], acc[t][j], 0, 0, 0);
    }
    // No barrier here: the next stage writes the other buffer, and its own barrier is
    // reached only once every wave has finished this stage.
  }

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
