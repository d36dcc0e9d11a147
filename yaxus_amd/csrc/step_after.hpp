// The step after the attention of a decode pass, on MI355X: the output projection
// (Backend::matmul with a bf16 weight, crates/yaxus-backend-cpu/src/lib.rs:234-248,
// 314-345: out[t][n] = x[t][:] . w[n][:], f32 activations, bf16 weight, f32 result) and
// the greedy pick over logits (SyncReadback::argmax_rows, lib.rs:432-440, 556-558).
//
// matmul_bf16_rows: weight-bandwidth-bound for decode row counts. A workgroup owns 16
// output columns (weight rows) and 16 activation rows; its 8 waves take eighths of K and
// their partial tiles are added in wave order (fixed, so the bits do not depend on
// timing). Per 32 k, one v_mfma_f32_16x16x32_bf16 per part of x: the weight is bf16
// exactly, and x goes in as three bf16 parts (hi, mid, lo: the 24 bits of an f32
// significand cut in three by truncation), so every product is exact and only the f32
// accumulation rounds. Range: exact for every finite x whose last significand bits stay
// within bf16's (= f32's) exponent range, i.e. |x| >= 2^-110; below that the low parts
// fall under the smallest subnormal (those x contribute below 2^-110 * |w| per term).
//   A (weight): lane (c, g) holds w[n0 + c][k + 8g .. k + 8g + 7]
//   B (x part): lane (c, g) holds x[t0 + c][k + 8g .. k + 8g + 7]
//   D: lane (c, g) holds out[t0 + c][n0 + 4g + i], i = 0..3
//
// argmax_rows: per row the first index of the largest value; NaN is never chosen and a
// row with nothing above -inf gives 0, as the CPU loop does (best starts at (0, -inf),
// replaced on a strictly larger value). Each value maps to a 64-bit key, (order-
// preserving bits of the value) << 32 | ~index, so the largest key is the largest value
// at its first index; workgroups reduce a slice each, and the last one of a row to
// arrive (an arrival counter, left at zero) reduces the slices' keys in slice order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_decode.hpp"

namespace yx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

static constexpr int kMmWaves = 8;
static constexpr int kMmSteps = 4;  // 32-wide k steps per wave and pass of its loop

// t rows of x [t][k] f32, w [n][k] bf16 bits, out [t][n] f32. Grid: (ceil(n / 16),
// ceil(t / 16), ks): the ks workgroups of an output tile take consecutive parts of k
// (whole 32-wide steps), their 8 waves eighths of those; k a multiple of 8
// (host-checked), n and t any. With ks > 1 each workgroup's tile goes to part (write-
// through) and the tile's last workgroup to arrive (counters, left at zero) adds the
// parts in k order.
__global__ __launch_bounds__(64 * kMmWaves) void matmul_bf16_rows(const float* __restrict__ x,
                                                                  const uint16_t* __restrict__ w,
                                                                  float* __restrict__ out, uint32_t t,
                                                                  uint32_t k, uint32_t n,
                                                                  f32x4* __restrict__ part,
                                                                  uint32_t part_bytes,
                                                                  uint32_t* __restrict__ counters) {
  __shared__ f32x4 wpart[kMmWaves][64];
  __shared__ uint32_t last;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  const uint32_t n0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
  const uint32_t ks = gridDim.z, kp = blockIdx.z;
  const uint32_t wn = n0 + c, xt = t0 + c;
  const bool wrow = wn < n, xrow = xt < t;
  // This wave's steps of 32 k (the last step may be partial: lanes past k read zeros).
  const uint32_t steps = (k + 31) / 32;
  const uint32_t p0 = steps * kp / ks, p1 = steps * (kp + 1) / ks;
  const uint32_t s0 = p0 + (p1 - p0) * wave / kMmWaves, s1 = p0 + (p1 - p0) * (wave + 1) / kMmWaves;
  const uint16_t* wp = w + static_cast<size_t>(wrow ? wn : 0) * k;
  const float* xp = x + static_cast<size_t>(xrow ? xt : 0) * k;
  f32x4 acc = {0, 0, 0, 0};
  for (uint32_t s = s0; s < s1; s += kMmSteps) {
    u16x8 wv[kMmSteps];
    f32x4 xa[kMmSteps], xb[kMmSteps];
#pragma unroll
    for (int u = 0; u < kMmSteps; ++u) {
      const uint32_t kk = (s + u) * 32 + 8 * g;
      const bool ok = (s + u < s1) & (kk < k);
      wv[u] = (ok & wrow) ? __builtin_nontemporal_load(reinterpret_cast<const u16x8*>(wp + kk))
                          : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      xa[u] = (ok & xrow) ? *reinterpret_cast<const f32x4*>(xp + kk) : f32x4{0, 0, 0, 0};
      xb[u] = (ok & xrow) ? *reinterpret_cast<const f32x4*>(xp + kk + 4) : f32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kMmSteps; ++u) {
      const float v[8] = {xa[u].x, xa[u].y, xa[u].z, xa[u].w, xb[u].x, xb[u].y, xb[u].z, xb[u].w};
      bf16x8 hi, mid, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // Truncated parts: hi = the top 8 significand bits, mid the next 8, lo the last
        // 8, each difference exact. A finite x never rounds up to inf (x near FLT_MAX),
        // and an infinite x is carried by hi alone (no inf - inf).
        const float xh = __uint_as_float(__float_as_uint(v[e]) & 0xffff0000u);
        const bool fin = __builtin_isfinite(v[e]);
        const float r1 = fin ? v[e] - xh : 0.0f;
        const float xm = __uint_as_float(__float_as_uint(r1) & 0xffff0000u);
        hi[e] = static_cast<__bf16>(xh);
        mid[e] = static_cast<__bf16>(xm);
        lo[e] = static_cast<__bf16>(r1 - xm);
      }
      const bf16x8 a = __builtin_bit_cast(bf16x8, wv[u]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, hi, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, mid, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, lo, acc, 0, 0, 0);
    }
  }
  wpart[wave][lane] = acc;
  __syncthreads();
  const size_t tile = static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x;
  f32x4 sum = {0, 0, 0, 0};
  if (wave == 0) {
    sum = wpart[0][lane];
#pragma unroll
    for (int wv = 1; wv < kMmWaves; ++wv) {
      const f32x4 q = wpart[wv][lane];
      sum = f32x4{sum.x + q.x, sum.y + q.y, sum.z + q.z, sum.w + q.w};
    }
    if (ks > 1)  // to memory all XCDs share (write-through) before the arrival
      st4_coherent(make_rsrc(part, part_bytes), static_cast<uint32_t>(((tile * ks + kp) * 64 + lane) * 16),
                   __builtin_bit_cast(float4, sum));
  }
  if (ks > 1) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t* cnt = counters + tile * kCounterStride;
      const uint32_t arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
      last = arrived == ks - 1;
      if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last || wave != 0) return;
    sum = f32x4{0, 0, 0, 0};
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, part_bytes);
    for (uint32_t q = 0; q < ks; ++q) {  // the parts in k order
      const f32x4 v = __builtin_bit_cast(f32x4, ld4_coherent(rp, static_cast<uint32_t>(((tile * ks + q) * 64 + lane) * 16)));
      sum = q == 0 ? v : f32x4{sum.x + v.x, sum.y + v.y, sum.z + v.z, sum.w + v.w};
    }
  } else if (wave != 0) {
    return;
  }
  if (xrow) {
    float* o = out + static_cast<size_t>(xt) * n + n0 + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n0 + 4 * g + i < n) o[i] = sum[i];
  }
}

// Order-preserving key of a value at an index: larger value, then smaller index, gives
// the larger key. NaN gets 0 (below every key of a number); -0 and +0 are one value.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t i) {
  if (v != v) return 0ull;
  const uint32_t b = v == 0.0f ? 0u : __builtin_bit_cast(uint32_t, v);
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<unsigned long long>(ord) << 32) | static_cast<uint32_t>(~i);
}

static constexpr int kArgmaxThreads = 256;
static constexpr int kArgmaxQuads = 8;  // 16-byte loads in flight per thread

// Grid: (slices, rows). keys [rows][slices] and counters [rows] are scratch (counters
// zero on entry, left at zero).
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows(const float* __restrict__ logits,
                                                              uint32_t cols, uint32_t* __restrict__ out,
                                                              unsigned long long* __restrict__ keys,
                                                              uint32_t* __restrict__ counters) {
  const uint32_t row = blockIdx.y, slice = blockIdx.x, nsl = gridDim.x;
  const uint32_t c0 = static_cast<uint32_t>(static_cast<uint64_t>(cols) * slice / nsl);
  const uint32_t c1 = static_cast<uint32_t>(static_cast<uint64_t>(cols) * (slice + 1) / nsl);
  const float* lr = logits + static_cast<size_t>(row) * cols;
  // The CPU's start: index 0 at -inf (a row of -inf and NaN gives 0).
  unsigned long long best = slice == 0 ? argmax_key(-INFINITY, 0) : 0ull;
  // Whole 16-byte quads of the slice (rows 16-byte aligned: the host checks cols % 4),
  // up to kArgmaxQuads per thread loaded before any is compared; the rest one by one.
  uint32_t i = c0;
  if ((cols & 3) == 0) {
    const uint32_t q0 = (c0 + 3) / 4, q1 = c1 / 4;
    for (uint32_t qb = q0; qb < q1; qb += kArgmaxQuads * kArgmaxThreads) {
      f32x4 v[kArgmaxQuads];
#pragma unroll
      for (int u = 0; u < kArgmaxQuads; ++u) {
        const uint32_t qq = qb + threadIdx.x + u * kArgmaxThreads;
        v[u] = qq < q1 ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(lr) + qq)
                       : f32x4{NAN, NAN, NAN, NAN};
      }
#pragma unroll
      for (int u = 0; u < kArgmaxQuads; ++u) {
        const uint32_t e = 4 * (qb + threadIdx.x + u * kArgmaxThreads);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const unsigned long long kk = argmax_key(v[u][j], e + j);
          best = kk > best ? kk : best;
        }
      }
    }
    // The values before the first and after the last whole quad.
    const uint32_t head = min(4 * q0, c1), tail = max(4 * q1, head);
    for (uint32_t e = c0 + threadIdx.x; e < head; e += kArgmaxThreads) {
      const unsigned long long kk = argmax_key(lr[e], e);
      best = kk > best ? kk : best;
    }
    i = tail;
  }
  for (i += threadIdx.x; i < c1; i += kArgmaxThreads) {
    const unsigned long long kk = argmax_key(__builtin_nontemporal_load(lr + i), i);
    best = kk > best ? kk : best;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off);
    best = o > best ? o : best;
  }
  __shared__ unsigned long long wbest[kArgmaxThreads / 64];
  __shared__ uint32_t last;
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = wbest[0];
    for (int wv = 1; wv < kArgmaxThreads / 64; ++wv) b = wbest[wv] > b ? wbest[wv] : b;
    if (nsl == 1) {
      out[row] = ~static_cast<uint32_t>(b);
      last = 0;
    } else {
      // The slice's key goes to memory all XCDs share (write-through) before the arrival
      // is counted; the row's last arrival reads the keys the same way.
      __hip_atomic_store(keys + static_cast<size_t>(row) * nsl + slice, b, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      uint32_t* cnt = counters + static_cast<size_t>(row) * kCounterStride;
      const uint32_t arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
      last = arrived == nsl - 1;
      if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!last) return;
  if (threadIdx.x < 64) {
    unsigned long long b = 0ull;
    for (uint32_t s = threadIdx.x; s < nsl; s += 64) {
      const unsigned long long kk = __hip_atomic_load(keys + static_cast<size_t>(row) * nsl + s,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      b = kk > b ? kk : b;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const unsigned long long o = __shfl_xor(b, off);
      b = o > b ? o : b;
    }
    if (threadIdx.x == 0) out[row] = ~static_cast<uint32_t>(b);
  }
}

}  // namespace yx
