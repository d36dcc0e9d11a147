// Per-head RMSNorm + half-split RoPE of a pass's queries and keys, with the keys and
// values stored at the rows' KV slots: `LayerPass::write_rows`
// (crates/yaxus-backend-cpu/src/lib.rs:359-385), the step before attention, which the
// reference GPU backend runs as QK_ROPE (crates/yaxus-backend-gpu/src/shaders.rs:285-341).
//
// One wave per (row, head) of the row's hq query heads and hkv key heads (the wave of a
// key head also stores that head's value). Lane j holds dims j and j + 64, the pair
// RoPE rotates together. The arithmetic is the CPU backend's, in its order, so the
// results carry the same bits:
//   sum of squares: one lane adds the 128 squares in dim order (rmsnorm_row, lib.rs:296-302);
//   r = 1 / sqrt(sum / 128 + eps) with correctly rounded division and square root;
//   y = (1 + w) * (x * r);
//   x[j] = a cos - b sin, x[j + 64] = b cos + a sin, with no fused multiply-add;
//   K rounded to binary16 (nearest even) into the arena's K order, V copied likewise.
// cos/sin come from a table [rope_len][64] cos then [rope_len][64] sin, computed on the
// host by the model's Rope::cos_sin (crates/yaxus-model/src/config.rs:213-219), as the
// reference GPU backend does (crates/yaxus-backend-gpu/src/ops/attention.rs:112-120).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_kernels.hpp"

namespace yx {

static constexpr int kRopeWaves = 4;

__global__ __launch_bounds__(64 * kRopeWaves) void qk_norm_rope_append(
    const float* __restrict__ qkv, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, const float* __restrict__ rope_cs, uint32_t rope_len,
    float eps, const uint32_t* __restrict__ pos, const uint32_t* __restrict__ kv_slot,
    _Float16* __restrict__ kc, _Float16* __restrict__ vc, float* __restrict__ q_out,
    uint32_t hq, uint32_t hkv, uint32_t page_size) {
#pragma clang fp contract(off)
  __shared__ float sq[kRopeWaves][128];
  const uint32_t row = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t h = blockIdx.y * kRopeWaves + wave;  // head: q heads, then key heads
  if (h >= hq + hkv) return;                          // whole wave
  const bool is_q = h < hq;
  const uint32_t qd = hq * 128, kvd = hkv * 128;
  const float* src = qkv + static_cast<size_t>(row) * (qd + 2 * kvd) + (is_q ? h * 128 : qd + (h - hq) * 128);
  const float x0 = src[lane], x1 = src[lane + 64];

  sq[wave][lane] = x0 * x0;
  sq[wave][lane + 64] = x1 * x1;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float ss = 0.0f;
  if (lane == 0)
    for (int i = 0; i < 128; ++i) ss += sq[wave][i];
  ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 0));
  const float r = 1.0f / __builtin_sqrtf(ss / 128.0f + eps);

  const float* w = is_q ? q_norm : k_norm;
  const float y0 = (1.0f + w[lane]) * (x0 * r);
  const float y1 = (1.0f + w[lane + 64]) * (x1 * r);
  const uint32_t p = pos[row];
  const float cs = rope_cs[static_cast<size_t>(p) * 64 + lane];
  const float sn = rope_cs[(static_cast<size_t>(rope_len) + p) * 64 + lane];
  const float ab = y0 * cs, bs = y1 * sn, bc = y1 * cs, as = y0 * sn;
  const float o0 = ab - bs;
  const float o1 = bc + as;

  if (is_q) {
    float* dst = q_out + static_cast<size_t>(row) * qd + h * 128;
    dst[lane] = o0;
    dst[lane + 64] = o1;
    return;
  }
  const uint32_t kh = h - hq;
  const uint32_t slot = kv_slot[row];
  const uint32_t off = slot % page_size;
  const size_t region = (static_cast<size_t>(slot / page_size) * hkv + kh) * page_size * 128;
  kc[region + k_offset(off, lane / 8) + lane % 8] = static_cast<_Float16>(o0);
  kc[region + k_offset(off, (lane + 64) / 8) + lane % 8] = static_cast<_Float16>(o1);
  const float* vsrc = src + kvd;  // the value head follows the key heads
  vc[region + off * 128 + lane] = static_cast<_Float16>(vsrc[lane]);
  vc[region + off * 128 + lane + 64] = static_cast<_Float16>(vsrc[lane + 64]);
}

}  // namespace yx
