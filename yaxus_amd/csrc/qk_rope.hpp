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
//   K rounded to binary16 (nearest even) into the arena's K order, V likewise (16-byte
//   stores of its row).
// cos/sin come from a table [rope_len][64] cos then [rope_len][64] sin, computed on the
// host by the model's Rope::cos_sin (crates/yaxus-model/src/config.rs:213-219), as the
// reference GPU backend does (crates/yaxus-backend-gpu/src/ops/attention.rs:112-120).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_kernels.hpp"

namespace yx {

static constexpr int kRopeWaves = 4;

// One wave, one head vector `src` (128 f32): RMSNorm with weights w (offset 1) and
// half-split RoPE at position p; returns this lane's results for dims lane and
// lane + 64. sq: 128 floats of LDS for this wave.
__device__ __forceinline__ void norm_rope_head(const float* __restrict__ src, const float* __restrict__ w,
                                               const float* __restrict__ rope_cs, uint32_t rope_len,
                                               uint32_t p, float eps, uint32_t lane, float* sq,
                                               float& o0, float& o1) {
#pragma clang fp contract(off)
  const float x0 = src[lane], x1 = src[lane + 64];
  sq[lane] = x0 * x0;
  sq[lane + 64] = x1 * x1;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float ss = 0.0f;
  if (lane == 0)
    for (int i = 0; i < 128; ++i) ss += sq[i];
  ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 0));
  const float r = 1.0f / __builtin_sqrtf(ss / 128.0f + eps);
  const float y0 = (1.0f + w[lane]) * (x0 * r);
  const float y1 = (1.0f + w[lane + 64]) * (x1 * r);
  const float cs = rope_cs[static_cast<size_t>(p) * 64 + lane];
  const float sn = rope_cs[(static_cast<size_t>(rope_len) + p) * 64 + lane];
  const float ab = y0 * cs, bs = y1 * sn, bc = y1 * cs, as = y0 * sn;
  o0 = ab - bs;
  o1 = bc + as;
}

// Stores one key head (k already normalised and rotated: lane's dims lane, lane + 64)
// and its raw value head `vsrc` (128 f32) at `slot`: binary16, nearest even.
__device__ __forceinline__ void store_kv_head(float k0, float k1, const float* __restrict__ vsrc,
                                              uint32_t slot, uint32_t kh, uint32_t hkv,
                                              uint32_t page_size, uint32_t lane, _Float16* kc,
                                              _Float16* vc) {
  const uint32_t off = slot % page_size;
  const size_t region = (static_cast<size_t>(slot / page_size) * hkv + kh) * page_size * 128;
  kc[region + k_offset(off, lane / 8) + lane % 8] = static_cast<_Float16>(k0);
  kc[region + k_offset(off, (lane + 64) / 8) + lane % 8] = static_cast<_Float16>(k1);
  if (lane < 16) {  // the value row: 16 lanes of 16 bytes
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const float4 a = *reinterpret_cast<const float4*>(vsrc + lane * 8);
    const float4 b = *reinterpret_cast<const float4*>(vsrc + lane * 8 + 4);
    *reinterpret_cast<h8*>(vc + region + off * 128 + lane * 8) =
        h8{static_cast<_Float16>(a.x), static_cast<_Float16>(a.y), static_cast<_Float16>(a.z),
           static_cast<_Float16>(a.w), static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
           static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
  }
}

__global__ __launch_bounds__(64 * kRopeWaves) void qk_norm_rope_append(
    const float* __restrict__ qkv, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, const float* __restrict__ rope_cs, uint32_t rope_len,
    float eps, const uint32_t* __restrict__ pos, const uint32_t* __restrict__ kv_slot,
    _Float16* __restrict__ kc, _Float16* __restrict__ vc, float* __restrict__ q_out,
    uint32_t hq, uint32_t hkv, uint32_t page_size) {
  __shared__ float sq[kRopeWaves][128];
  const uint32_t row = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t h = blockIdx.y * kRopeWaves + wave;  // head: q heads, then key heads
  if (h >= hq + hkv) return;                          // whole wave
  const bool is_q = h < hq;
  const uint32_t qd = hq * 128, kvd = hkv * 128;
  const float* src = qkv + static_cast<size_t>(row) * (qd + 2 * kvd) + (is_q ? h * 128 : qd + (h - hq) * 128);
  float o0, o1;
  norm_rope_head(src, is_q ? q_norm : k_norm, rope_cs, rope_len, pos[row], eps, lane, sq[wave], o0, o1);
  if (is_q) {
    float* dst = q_out + static_cast<size_t>(row) * qd + h * 128;
    dst[lane] = o0;
    dst[lane + 64] = o1;
    return;
  }
  // The value head follows the key heads.
  store_kv_head(o0, o1, src + kvd, kv_slot[row], h - hq, hkv, page_size, lane, kc, vc);
}

}  // namespace yx
