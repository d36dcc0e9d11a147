// Per-head RMSNorm + half-split RoPE of a pass's queries and keys, with the keys and
// values stored at the rows' KV slots: `LayerPass::write_rows`
// (crates/yaxus-backend-cpu/src/lib.rs:359-385), the step before attention, which the
// reference GPU backend runs as QK_ROPE (crates/yaxus-backend-gpu/src/shaders.rs:285-341).
//
// Lane j of a wave holds dims j and j + 64 of a head, the pair RoPE rotates together
// (a key head's wave also stores that head's value). The arithmetic is the CPU
// backend's, in its order, so the results carry the same bits:
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
// and its raw value head `vsrc` (128 f32) at `slot` (pages of 1 << page_shift slots):
// binary16, nearest even.
__device__ __forceinline__ void store_kv_head(float k0, float k1, const float* __restrict__ vsrc,
                                              uint32_t slot, uint32_t kh, uint32_t hkv,
                                              uint32_t page_shift, uint32_t lane, _Float16* kc,
                                              _Float16* vc) {
  const uint32_t off = slot & ((1u << page_shift) - 1u);
  const size_t region = ((static_cast<size_t>(slot >> page_shift) * hkv + kh) * 128) << page_shift;
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

// The same into an f32 arena (`[page][kv_head][page_size][128]`, K like V): stored as
// computed.
__device__ __forceinline__ void store_kv_head(float k0, float k1, const float* __restrict__ vsrc,
                                              uint32_t slot, uint32_t kh, uint32_t hkv,
                                              uint32_t page_shift, uint32_t lane, float* kc,
                                              float* vc) {
  const uint32_t off = slot & ((1u << page_shift) - 1u);
  const size_t row = (((static_cast<size_t>(slot >> page_shift) * hkv + kh) * 128) << page_shift) + off * 128;
  kc[row + lane] = k0;
  kc[row + lane + 64] = k1;
  if (lane < 32)  // the value row: 32 lanes of 16 bytes
    *reinterpret_cast<float4*>(vc + row + lane * 4) = *reinterpret_cast<const float4*>(vsrc + lane * 4);
}

// write_rows over a whole pass: the pass's head vectors (per row its hq query heads,
// then its hkv key heads, or the key heads only; vector i = row i / heads) in
// workgroups of kRopeVecs.
// Each workgroup stages its vectors in LDS (coalesced: a row's q and k heads are
// contiguous in qkv), then lanes of one wave add each vector's 128 squares serially in
// dim order, one lane per vector (the CPU backend's order, so the same bits; a wave per
// vector with one lane adding, as the decode kernel does for its few rows, leaves 63 of
// 64 lanes idle), and then the four waves normalise, rotate and store, a lane per dim
// pair (j, j + 64). Rows of 129 floats keep the serial reads free of bank conflicts.
// Small workgroups keep many in flight: the per-workgroup chain of loads and the
// serial sum, not the arithmetic, sets the time.
static constexpr int kRopeVecs = 16;  // 16: 18.0 us at 4096 rows; 32: 19.1; 64: 24.6
static constexpr int kRopeThreads = 256;

// T: the arena's element type (_Float16 or float).
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void qk_norm_rope_append(
    const float* __restrict__ qkv, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, const float* __restrict__ rope_cs, uint32_t rope_len,
    float eps, const uint32_t* __restrict__ pos, const uint32_t* __restrict__ kv_slot,
    T* __restrict__ kc, T* __restrict__ vc, float* __restrict__ q_out,
    uint32_t hq, uint32_t hkv, uint32_t page_shift, uint32_t nvec, uint32_t first) {
#pragma clang fp contract(off)
  __shared__ float xs[kRopeVecs][129];
  __shared__ float rs[kRopeVecs];
  // first = 0: every head; first = hq: the key heads only (the caller normalises the
  // query heads itself). nh heads per row from head `first` on.
  const uint32_t nh = hq + hkv - first, qd = hq * 128, kvd = hkv * 128, cols = qd + 2 * kvd;
  const uint32_t v0 = blockIdx.x * kRopeVecs;
  const uint32_t t = threadIdx.x, j = t & 63;
  // Vector v0 + m is head (h0 + m) % nh of row row0 + (h0 + m) / nh; m < kRopeVecs.
  const uint32_t row0 = v0 / nh, h0 = v0 - row0 * nh;
  const float inv_nh = 1.0f / static_cast<float>(nh);
  auto split = [&](uint32_t m, uint32_t& row, uint32_t& h) {
    const uint32_t x = h0 + m;  // below kRopeVecs + nh: the float quotient is off by at most one
    uint32_t d = static_cast<uint32_t>(static_cast<float>(x) * inv_nh);
    if (d * nh > x) --d;
    else if ((d + 1) * nh <= x) ++d;
    row = row0 + d;
    h = first + x - d * nh;
  };
  constexpr int kPer = kRopeVecs / (kRopeThreads / 64);  // vectors per thread in the last step
  constexpr int kStage = kRopeVecs * 32 / kRopeThreads;    // float4 per thread when staging
  // Loads in the order their results are needed, so that one chain (positions, then
  // their cos/sin) overlaps the other (the vectors, then their sums): positions, the
  // vectors, then cos/sin, slots and weights.
  uint32_t prow[kPer], pslot[kPer];
  float pcs[kPer], psn[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t m = (t >> 6) + i * (kRopeThreads / 64);
    uint32_t h;
    split(m, prow[i], h);
    if (v0 + m >= nvec) prow[i] = 0;
    pslot[i] = pos[prow[i]];
  }
  float4 stage[kStage];
#pragma unroll
  for (int k = 0; k < kStage; ++k) {
    const uint32_t idx = k * kRopeThreads + t, v = idx / 32, c4 = idx % 32;
    uint32_t row, h;
    split(v, row, h);
    if (v0 + v >= nvec) row = h = 0;
    // The key heads follow the query heads in a row: vector h starts at h * 128.
    stage[k] = *reinterpret_cast<const float4*>(qkv + static_cast<size_t>(row) * cols + h * 128 + c4 * 4);
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    pcs[i] = rope_cs[static_cast<size_t>(pslot[i]) * 64 + j];
    psn[i] = rope_cs[(static_cast<size_t>(rope_len) + pslot[i]) * 64 + j];
    pslot[i] = kv_slot[prow[i]];
  }
  const float qw0 = 1.0f + q_norm[j], qw1 = 1.0f + q_norm[j + 64];
  const float kw0 = 1.0f + k_norm[j], kw1 = 1.0f + k_norm[j + 64];
#pragma unroll
  for (int k = 0; k < kStage; ++k) {
    const uint32_t idx = k * kRopeThreads + t, v = idx / 32, c4 = idx % 32;
    xs[v][c4 * 4] = stage[k].x;
    xs[v][c4 * 4 + 1] = stage[k].y;
    xs[v][c4 * 4 + 2] = stage[k].z;
    xs[v][c4 * 4 + 3] = stage[k].w;
  }
  __syncthreads();
  if (t < kRopeVecs) {  // one vector per lane of wave 0, its squares added in dim order
    float ss = 0.0f;
#pragma unroll
    for (int i0 = 0; i0 < 128; i0 += 32) {
      float x[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) x[i] = xs[t][i0 + i];
#pragma unroll
      for (int i = 0; i < 32; ++i) ss += x[i] * x[i];
    }
    rs[t] = 1.0f / __builtin_sqrtf(ss / 128.0f + eps);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t m = (t >> 6) + i * (kRopeThreads / 64), gv = v0 + m;
    if (gv >= nvec) break;
    uint32_t row, h;
    split(m, row, h);
    const bool is_q = h < hq;
    const float r = rs[m];
    const float y0 = (is_q ? qw0 : kw0) * (xs[m][j] * r);
    const float y1 = (is_q ? qw1 : kw1) * (xs[m][j + 64] * r);
    const float ab = y0 * pcs[i], bs = y1 * psn[i], bc = y1 * pcs[i], as = y0 * psn[i];
    const float o0 = ab - bs, o1 = bc + as;
    if (is_q) {
      float* dst = q_out + static_cast<size_t>(row) * qd + h * 128;
      dst[j] = o0;
      dst[j + 64] = o1;
    } else {
      store_kv_head(o0, o1, qkv + static_cast<size_t>(row) * cols + qd + kvd + (h - hq) * 128,
                    pslot[i], h - hq, hkv, page_shift, j, kc, vc);
    }
  }
}

}  // namespace yx
