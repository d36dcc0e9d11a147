// Paged prefill / chunked-prefill attention over the f32 arena (the reference's own K/V
// precision, crates/yaxus-backend-cpu/src/lib.rs:205-214): the same arithmetic as
// `LayerPass::attend` (crates/yaxus-backend-cpu/src/lib.rs:389-427) for passes with many
// rows per sequence, with exact f32 products (v_mfma_f32_16x16x4_f32) and f32
// accumulation, so no operand is rounded to a narrower type and every finite f32 K/V
// value the reference accepts is served.
//
// Work items are built as for the f16 prefill kernel, with kPf32Rows = 128 logical rows
// (consecutive rows of one sequence, all query heads of one KV head) per workgroup of 8
// waves, 16 columns per wave. Keys stream from HBM into a 4-slot LDS ring of 32-key stages (two blocks of 16;
// global_load_lds_dwordx4, three stages in flight while one is computed), laid out in
// operand order so that every LDS read is one contiguous 1 KiB per wave. Per block of 16
// keys and wave:
//   S^T[key][col] = K . Q^T     32 x v_mfma_f32_16x16x4_f32 (dims in steps of 4)
//   online softmax per column (permlane swaps across the 4 lane groups)
//   O^T += V^T P^T              32 x v_mfma_f32_16x16x4_f32 (keys in steps of 4)
// Operand layouts (lane l, c = l % 16, g = l / 16), those of the f32 decode kernel:
//   QK step 4t + e: lane holds K[key c][16t + 4g + e] and q[col c][16t + 4g + e];
//     S^T[key 4g + i][col c] is element i of the sum of the four step-parity
//     accumulators.
//   PV step (t, m): lane holds V[key 4g + t][64(m / 4) + 4c + m % 4] (A) and
//     P[key 4g + t][col c] (B); O lands as dims 64h + 16g + 4i + (0..3) of column c
//     in elements i of accumulators 4h .. 4h + 3.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_prefill.hpp"

namespace yx {

// Two shapes: 8 waves (128 logical rows) with a 4-stage ring, one workgroup per CU; or
// 4 waves (64 rows) with a 2-stage ring (64 KiB), two workgroups per CU, for passes
// whose sequences have few rows (a tile of 128 would leave most of its waves idle).
template <int W>
struct Pf32Shape {
  static constexpr int kRows = W * 16;             // logical rows per work item (one tile per wave)
  static constexpr int kRing = W == 8 ? 4 : 2;     // LDS stages (32 KiB each)
  static constexpr int kLead = kRing - 1;          // stages in flight ahead of the one computed
  static constexpr int kRowsPerWave = 32 / W;      // stage rows (1 KiB each) each wave moves
};
static constexpr int kPf32Waves = 8;
static constexpr int kPf32Rows = Pf32Shape<8>::kRows;
static constexpr int kPf32SmallRows = Pf32Shape<4>::kRows;

template <int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2))) void paged_attn_prefill_f32(
    const PrefillItem* __restrict__ items, const uint32_t* pos,
    const uint32_t* __restrict__ pages, const float* __restrict__ kc, const float* __restrict__ vc,
    const float* q, float* __restrict__ out, uint32_t hq, uint32_t hkv, uint32_t bpp_shift,
    uint32_t window, float scale_log2, float* __restrict__ part_o, float2* __restrict__ part_ml,
    uint32_t* __restrict__ counters, uint32_t part_o_bytes, uint32_t part_ml_bytes) {
  // A ring of stages; each is 32 rows of 1 KiB: K of block b as rows 8b + t ([t][g][key c],
  // float4 = K[c][16t + 4g .. + 3]), then V of block b as rows 16 + 8b + 2t + h
  // ([t][h][g][c], float4 = V[4g + t][64h + 4c .. + 3]).
  using S = Pf32Shape<W>;
  constexpr int kRing = S::kRing, kLead = S::kLead, kRpw = S::kRowsPerWave;
  __shared__ float4 ring[kRing][32 * 64];
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
  const uint32_t nblk = it.blk1 - it.blk0;
  const uint32_t nst = (nblk + 1) / 2;  // stages of two blocks

  // Wave w moves stage rows kRpw * w .. kRpw * (w + 1) - 1, all of one block's K (rows
  // 0-15) or V (rows 16-31).
  const int row0 = wave * kRpw;
  const bool my_v = row0 >= 16;
  const uint32_t my_blk = static_cast<uint32_t>((row0 & 15) >> 3);
  uint32_t src_off[kRpw];  // bytes within the block, per row
#pragma unroll
  for (int r = 0; r < kRpw; ++r) {
    const int row = (row0 & 7) + r;  // row within the block's 8 rows
    if (!my_v)
      src_off[r] = static_cast<uint32_t>((c * kD + 16 * row + 4 * g) * 4);
    else
      src_off[r] = static_cast<uint32_t>(((4 * g + (row >> 1)) * kD + 64 * (row & 1) + 4 * c) * 4);
  }
  const uint32_t ring_base = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) float4*)&ring[0][0]));
  // Page of the block the wave moves for stage st, read one stage ahead.
  auto page_of = [&](uint32_t st) __attribute__((always_inline)) {
    uint32_t b = it.blk0 + st * 2 + my_blk;
    b = b < it.blk1 ? b : it.blk1 - 1;  // past the end: re-read the last block (unused)
    return uint2{pt[b >> bpp_shift], b & bpp_mask};
  };
  uint2 next_page = page_of(0);
  auto issue = [&](uint32_t st) __attribute__((always_inline)) {
    const size_t elem = (static_cast<size_t>(next_page.x) * hkv + kh) * head_stride +
                        static_cast<size_t>(next_page.y) * 16 * kD;
    next_page = page_of(st + 1);
    const char* blk = reinterpret_cast<const char*>((my_v ? vc : kc) + elem);
    const uint32_t dst = ring_base + (st & (kRing - 1)) * (32 * 1024) + static_cast<uint32_t>(row0) * 1024u;
#pragma unroll
    for (int r = 0; r < kRpw; ++r) load_to_lds16(blk + src_off[r], dst + r * 1024);
  };

  // This lane's column: its row position, key window and q (dims 16t + 4g + 0..3) as
  // given; the summed products are scaled into log2 units once, per score.
  const uint32_t lr = wave * 16 + c;
  const bool has = lr < nlog;
  const uint32_t lrc = has ? lr : 0;
  const uint32_t rr = it.r0 + lrc / G, h = kh * G + lrc % G;
  const int p0 = static_cast<int>(pos[rr]);
  const int rpos = has ? p0 : -1;
  const int rlo = (window > 0 && p0 + 1 > static_cast<int>(window)) ? p0 + 1 - static_cast<int>(window) : 0;
  float4 qv[8];
  {
    const float* qp = q + (static_cast<size_t>(rr) * hq + h) * kD + 4 * g;
#pragma unroll
    for (int t = 0; t < 8; ++t) qv[t] = *reinterpret_cast<const float4*>(qp + 16 * t);
  }
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < kLead; ++j) issue(j);
#pragma unroll
  for (int t = 0; t < 8; ++t)
    if (!has) qv[t] = float4{0, 0, 0, 0};

  // The wave's key range: blocks [wa, wb) hold a key some column of the wave sees.
  int mx = rpos, lo = has ? rlo : INT32_MAX, mn = rpos, hl = rlo;
#pragma unroll
  for (int s = 1; s < 16; s <<= 1) {
    mx = max(mx, __shfl_xor(mx, s));
    lo = min(lo, __shfl_xor(lo, s));
    mn = min(mn, __shfl_xor(mn, s));
    hl = max(hl, __shfl_xor(hl, s));
  }
  const int wmax = __builtin_amdgcn_readfirstlane(mx);
  const int wlo = __builtin_amdgcn_readfirstlane(lo);
  const int tmin = __builtin_amdgcn_readfirstlane(mn);  // -1 when the tile has an empty column
  const int tlo = __builtin_amdgcn_readfirstlane(hl);
  const int first_key = static_cast<int>(it.blk0 * 16);
  const int key_end = static_cast<int>(it.blk1 * 16);

  // As in the f16 kernel, the running maximum starts at a finite floor: masked scores
  // (-inf) give P = 0 and a column's first key rescales its zero state away.
  constexpr float kFloor = -1.0e30f;
  float m = kFloor, lsum = 0.0f;
  floatx4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = floatx4{0, 0, 0, 0};

  auto block = [&](auto masked, const float4* kb, const float4* vb, int key0) __attribute__((always_inline)) {
    float4 kf[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) kf[t] = kb[t * 64 + lane];
    floatx4 sp[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      sp[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t].x, qv[t].x, sp[0], 0, 0, 0);
      sp[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t].y, qv[t].y, sp[1], 0, 0, 0);
      sp[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t].z, qv[t].z, sp[2], 0, 0, 0);
      sp[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t].w, qv[t].w, sp[3], 0, 0, 0);
    }
    float4 vf[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) vf[r] = vb[r * 64 + lane];
    float x[4], bmax = kFloor;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s = ((sp[0][i] + sp[1][i]) + (sp[2][i] + sp[3][i])) * scale_log2;
      if constexpr (decltype(masked)::value) {
        const int kp = key0 + 4 * g + i;
        const bool ok = (kp >= rlo) & (kp <= rpos) & (kp < key_end);
        x[i] = ok ? s : -INFINITY;
      } else {
        x[i] = s;
      }
      bmax = fmaxf(bmax, x[i]);
    }
    const float mnew = fmaxf(m, max_xor32(max_xor16(bmax)));
    if (__builtin_amdgcn_ballot_w64(mnew > m + kLazyRescale)) {  // wave-uniform
      const float corr = __builtin_amdgcn_exp2f(m - mnew);
      lsum *= corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= corr;
      m = mnew;
    }
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = __builtin_amdgcn_exp2f(x[i] - m);
      lsum += pr[i];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) {
        const float4 vv = vf[2 * t + mm / 4];
        const float a = (mm % 4 == 0) ? vv.x : (mm % 4 == 1) ? vv.y : (mm % 4 == 2) ? vv.z : vv.w;
        acc[mm] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, pr[t], acc[mm], 0, 0, 0);
      }
    }
  };

  for (uint32_t st = 0; st < nst; ++st) {
    // This wave's loads of stage st are done when at most the kLead - 1 later stages'
    // are in flight; the barrier makes every wave's rows visible, and every wave has
    // finished computing stage st - 1, whose slot stage st + kLead refills.
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(kRpw * (kLead - 1)) : "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    issue(st + kLead);
    const float4* sb = &ring[st & (kRing - 1)][0];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int key0 = first_key + static_cast<int>(st * 32 + b * 16);
      if (key0 > wmax || key0 + 15 < wlo || key0 >= key_end) continue;  // wave-uniform
      const bool whole = (key0 + 15 <= tmin) & (key0 >= tlo) & (key0 + 16 <= key_end);
      if (whole)
        block(std::false_type{}, sb + b * 8 * 64, sb + (16 + b * 8) * 64, key0);
      else
        block(std::true_type{}, sb + b * 8 * 64, sb + (16 + b * 8) * 64, key0);
    }
  }
  // No load into LDS may land after the workgroup ends.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const float l = sum_xor32(sum_xor16(lsum));
  const uint32_t nch = it.chunk_nch >> 16;
  if (nch <= 1) {
    if (!has) return;
    float* o = out + (static_cast<size_t>(rr) * hq + h) * kD;
    const float inv = 1.0f / l;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(o + 64 * hh + 16 * g + 4 * i) =
            float4{acc[4 * hh][i] * inv, acc[4 * hh + 1][i] * inv, acc[4 * hh + 2][i] * inv,
                   acc[4 * hh + 3][i] * inv};
    return;
  }
  // A split tile: partials and the last chunk's merge, as in the binary16 kernel.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(part_o, part_o_bytes);
  const __amdgpu_buffer_rsrc_t rml = make_rsrc(part_ml, part_ml_bytes);
  if (has) {
    const size_t slot = (static_cast<size_t>(it.part_base) + (it.chunk_nch & 0xffffu)) * hkv + kh;
    const size_t e = slot * S::kRows + lr;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4_coherent(ro, static_cast<uint32_t>((e * kD + 64 * hh + 16 * g + 4 * i) * 4),
                     float4{acc[4 * hh][i], acc[4 * hh + 1][i], acc[4 * hh + 2][i], acc[4 * hh + 3][i]});
    if (g == 0) st2_coherent(rml, static_cast<uint32_t>(e * 8), float2{m, l});
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
  merge_tile<64 * W, S::kRows>(it.r0, it.nrows, it.part_base, nch, kh, G, hq, hkv, out, ro, rml);
}

}  // namespace yx
