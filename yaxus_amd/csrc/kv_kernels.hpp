// K/V store, page copy and data-fill kernels for the paged arena.
//
// Arena layout per layer, f32: K and V both `[page][kv_head][page_size][128]`.
// Arena layout per layer, binary16: V is `[page][kv_head][page_size][128]`; K is the
// same but each 16-key block of a (page, kv head) is stored `[4][16 keys][32 dims]`:
// dim d of key k of the block sits at (d / 32) * 512 + k * 32 + d % 32. That is the
// order in which the attention kernel's MFMA operand loads read it (1 KiB contiguous
// per load instruction).

#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace yx {

// Offset in halves of (key `off` of a page, dim chunk `ch` of 8 dims) within a
// (page, kv head) region of K.
__host__ __device__ inline size_t k_offset(uint32_t off, uint32_t ch) {
  return static_cast<size_t>(off / 16) * 2048 + (ch / 4) * 512 + (off % 16) * 32 + (ch % 4) * 8;
}

// The K/V store of write_rows (crates/yaxus-backend-cpu/src/lib.rs:378-383): one
// thread per 8 consecutive dims of one (row, kv head); two 16-byte f32 loads, a
// round-to-nearest-even conversion, one 16-byte store. blockIdx.y: 0 = K, 1 = V.
// 16 consecutive threads write one key's 256 bytes (V: one contiguous row; K: four
// contiguous 64-byte pieces).
__global__ __launch_bounds__(256) void kv_append_f16(const float* __restrict__ k,
                                                     const float* __restrict__ v,
                                                     const uint32_t* __restrict__ kv_slot,
                                                     _Float16* __restrict__ kc,
                                                     _Float16* __restrict__ vc, uint32_t rows,
                                                     uint32_t hkv, uint32_t page_size) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t per_row = hkv * 16;
  if (tid >= rows * per_row) return;
  const uint32_t row = tid / per_row, rem = tid % per_row, h = rem / 16, ch = rem % 16;
  const float* src = (blockIdx.y == 0 ? k : v) + (static_cast<size_t>(row) * hkv + h) * 128 + ch * 8;
  const uint32_t slot = kv_slot[row];
  const uint32_t page = slot / page_size, off = slot % page_size;
  const size_t region = (static_cast<size_t>(page) * hkv + h) * page_size * 128;
  _Float16* dst = blockIdx.y == 0 ? kc + region + k_offset(off, ch) : vc + region + off * 128 + ch * 8;
  const float4 a = *reinterpret_cast<const float4*>(src);
  const float4 b = *reinterpret_cast<const float4*>(src + 4);
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 o = {static_cast<_Float16>(a.x), static_cast<_Float16>(a.y), static_cast<_Float16>(a.z),
          static_cast<_Float16>(a.w), static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
          static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
  *reinterpret_cast<h8*>(dst) = o;
}

// The same store into an f32 arena (K and V both `[page][kv_head][page_size][128]`):
// one thread per 4 consecutive dims of one (row, kv head), a 16-byte copy.
__global__ __launch_bounds__(256) void kv_append_f32(const float* __restrict__ k,
                                                     const float* __restrict__ v,
                                                     const uint32_t* __restrict__ kv_slot,
                                                     float* __restrict__ kc, float* __restrict__ vc,
                                                     uint32_t rows, uint32_t hkv, uint32_t page_size) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t per_row = hkv * 32;
  if (tid >= rows * per_row) return;
  const uint32_t row = tid / per_row, rem = tid % per_row, h = rem / 32, ch = rem % 32;
  const float* src = (blockIdx.y == 0 ? k : v) + (static_cast<size_t>(row) * hkv + h) * 128 + ch * 4;
  const uint32_t slot = kv_slot[row];
  const uint32_t page = slot / page_size, off = slot % page_size;
  float* dst = (blockIdx.y == 0 ? kc : vc) + (static_cast<size_t>(page) * hkv + h) * page_size * 128 +
               off * 128 + ch * 4;
  *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(src);
}

// Plain streaming copy (also the calibration kernel for HBM byte counters).
__global__ __launch_bounds__(256) void dev_copy16(uint4* __restrict__ d,
                                                  const uint4* __restrict__ s, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    d[i] = s[i];
}

// XOR of every 8-byte word of a buffer (n 16-byte pieces): a read-only pass over the
// buffer (the read-side reference point for the HBM byte counters) and an
// order-independent checksum of device data.
__global__ __launch_bounds__(256) void dev_checksum16(const uint4* __restrict__ s, size_t n,
                                                      unsigned long long* out) {
  unsigned long long x = 0;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    typedef uint32_t w4 __attribute__((ext_vector_type(4)));
    const w4 v = __builtin_nontemporal_load(reinterpret_cast<const w4*>(s) + i);
    x ^= (static_cast<unsigned long long>(v.y) << 32 | v.x) ^ (static_cast<unsigned long long>(v.w) << 32 | v.z);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off);
  __shared__ unsigned long long part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) atomicXor(out, part[0] ^ part[1] ^ part[2] ^ part[3]);
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// N(0,1) fill: pair k uses u1 = top 53 bits of splitmix64(seed + 2k), u2 of
// splitmix64(seed + 2k + 1); r = sqrt(-2 ln(1 - u1)), th = 2 pi u2; element 2k is
// r cos th, element 2k + 1 is r sin th (computed in f64, rounded to the dtype).
__global__ __launch_bounds__(256) void fill_normal(void* __restrict__ dst, size_t n, int f16,
                                                   uint64_t seed, uint64_t offset) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const uint64_t e = offset + i, k = e >> 1;
    const double u1 = static_cast<double>(splitmix64(seed + 2 * k) >> 11) * 0x1.0p-53;
    const double u2 = static_cast<double>(splitmix64(seed + 2 * k + 1) >> 11) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log(1.0 - u1));
    const double th = 6.283185307179586 * u2;
    const float x = static_cast<float>((e & 1) ? r * sin(th) : r * cos(th));
    if (f16)
      static_cast<_Float16*>(dst)[i] = static_cast<_Float16>(x);
    else
      static_cast<float*>(dst)[i] = x;
  }
}

}  // namespace yx
