// Paged decode / verify attention for gfx950 (wave64, MFMA).
//
// Restates the arithmetic of `LayerPass::attend` (crates/yaxus-backend-cpu/src/
// lib.rs:389-427): per (row, query head), keys `[lo, pos]` of the row's sequence
// through its page table, softmax of q.k * scale, and the weighted sum of V. The
// reference GPU splits keys into chunks and merges them afterwards (ATTN_SPLIT +
// ATTN_COMBINE, crates/yaxus-backend-gpu/src/shaders.rs:1466-1637); here too, but the
// merge runs in the same kernel: the last work item of a (rows, kv head) to finish
// merges all chunks, in chunk order, so results do not depend on arrival order.
//
// Work item = (a group of consecutive rows of one sequence, one KV head, one chunk of
// 16-key blocks), one workgroup of W waves; the waves split the chunk's blocks and
// merge through LDS. The group's (row, query head) pairs are "logical rows". Three
// kernels below: the 8-row-tile kernels (`paged_attn_decode`, and the queue-balanced
// one-tile `paged_attn_decode_balanced`) and the 16-row-tile one
// (`paged_attn_decode_wide`), plus the f32-arena kernel at the end. In the 8-row
// tiles, NT tiles of 8 logical rows each sit in MFMA columns as an f16 hi part
// (columns 0-7) and an f16 lo part (columns 8-15) of q, so q.k keeps ~2^-22 relative
// accuracy with f16 K exact and f32 accumulation. Per block of 16 keys:
//   S^T[key][col] = K[key][:] . Q[col][:]         4 x v_mfma_f32_16x16x32_f16
//   online softmax per column; P = exp2(S*scale*log2e - m) split into hi/lo f16
//   O^T[dim][col] += V^T[dim][key] P^T[key][col]  8 x v_mfma_f32_16x16x32_f16 per 2 blocks
// Operand layouts (lane l, c = l % 16, g = l / 16):
//   K: A operand of QK, lane holds key c, dims p*32 + g*8 + 0..7 for MFMA p. The arena
//      stores each 16-key block of K as [p][key][32 dims] (see kv_kernels.hpp), so the
//      64 lanes' 16-byte loads of one MFMA read 1 KiB contiguous.
//   V: A operand of PV, lane holds dims c*8 + j of keys 4g..4g+3; V rows are stored
//      plainly ([key][128 dims]), so each of the 4 loads reads 4 rows contiguous.
//   The PV output lands as 32 consecutive dims (32g..32g+31) of column c per lane.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_kernels.hpp"
#include "qk_rope.hpp"

namespace yx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// One split-K work item (host-built, see runtime.hip).
struct AttnItem {
  uint32_t r0;         // first pass row of the group
  uint32_t nrows;      // rows in the group
  uint32_t pt_off;     // offset of the group's page table in the pass's pages
  uint32_t blk0;       // first 16-key block (absolute key / 16) of this chunk
  uint32_t blk1;       // one past the last block of this chunk
  uint32_t chunk;      // chunk index within the group
  uint32_t nch;        // chunks of the group (at most kMaxChunks)
  uint32_t part_base;  // first partial slot of the group
  uint32_t counter;    // arrival counter index of the group
  // Shared-prefix (cascade) passes. A prefix item (pref_info has kPrefixItem) attends
  // keys that every row of a run of consecutive groups shares (the same pages) for all
  // of their rows at once: pref_base / pref_nch then index its member groups in the
  // member list. A member group's items carry pref_base / pref_nch = the first partial
  // slot and chunk count of its prefix items and pref_info = the group's first row's
  // offset within them; its merge takes the prefix chunks first, then its own.
  uint32_t pref_base;
  uint32_t pref_nch;   // 0: no shared prefix
  uint32_t pref_info;
};
static constexpr uint32_t kPrefixItem = 0x80000000u;

// A member group of a shared prefix, for the prefix items' hand-off.
struct SubRef {
  uint32_t r0, nrows;      // the group's rows
  uint32_t part_base, nch;  // its own chunks' partial slots
  uint32_t counter;         // its arrival counter
  uint32_t row_off;         // its first row's offset among the prefix items' rows
  uint32_t pad[2];
};

static constexpr float kLog2e = 1.4426950408889634f;
static constexpr int kD = 128;
static constexpr uint32_t kMaxChunks = 256;
// Arrival counters (split-K hand-offs) sit one per 128-byte line, in uint32 units:
// atomics to one line queue behind each other at its L2 channel.
static constexpr uint32_t kCounterStride = 32;

// Lane l reads lane l^8 (DPP row rotate by 8 within each row of 16 lanes).
__device__ __forceinline__ float xor8(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
}

// Reductions over lanes l and l^16, or l and l^32, for every lane: the gfx950 permlane
// swaps exchange rows of 16 (or halves of 32) lanes between two registers in the VALU,
// without the LDS round trip of a swizzle or bpermute. With both registers holding the
// same value, each lane ends up with its own value in one and its partner's in the
// other; max and + are commutative, so both lanes of a pair get the same bits. Written
// as inline asm: the compiler's builtin for the swap treats the two results of a swap
// of equal inputs as equal, which they are not across lanes. The s_nop covers the
// wait states a swap needs after a VALU write of its operands.
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  __asm__("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  __asm__("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float max_xor16(float x) {
  float a = x, b = x;
  permlane16_swap(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float x) {
  float a = x, b = x;
  permlane32_swap(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor16(float x) {
  float a = x, b = x;
  permlane16_swap(a, b);
  return a + b;
}
__device__ __forceinline__ float sum_xor32(float x) {
  float a = x, b = x;
  permlane32_swap(a, b);
  return a + b;
}

// Write-through 16-byte store / coherent load of split-K partials through a buffer
// resource with the sc1 cache policy: the data goes to (and comes from) the memory
// all XCDs share, so the hand-off between workgroups needs no L2 write-back.
static constexpr int kCoherent = 16;  // sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ void st4_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, static_cast<int>(off), 0, kCoherent);
}
__device__ __forceinline__ float4 ld4_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, kCoherent));
}
__device__ __forceinline__ void st2_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, float2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, static_cast<int>(off), 0, kCoherent);
}
__device__ __forceinline__ float2 ld2_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, kCoherent));
}

// K/V of one 16-key block held by a lane (see the header comment for the mapping).
struct BlockRegs {
  half8 k[4];
  half8 v[4];
};

// kblk / vblk: the block's first half in the arena (2048 halves per block and head).
__device__ __forceinline__ void load_block(BlockRegs& r, const _Float16* __restrict__ kblk,
                                           const _Float16* __restrict__ vblk, int lane) {
  const int c = lane & 15, g = lane >> 4;
  const half8* kp = reinterpret_cast<const half8*>(kblk) + c * 4 + g;  // [p][key c][g]
#pragma unroll
  for (int p = 0; p < 4; ++p) r.k[p] = __builtin_nontemporal_load(kp + p * 64);
  const half8* vp = reinterpret_cast<const half8*>(vblk + (4 * g) * kD + c * 8);
#pragma unroll
  for (int i = 0; i < 4; ++i) r.v[i] = __builtin_nontemporal_load(vp + i * (kD / 8));
}

// Waves per workgroup (W): they share one work item's blocks and merge through LDS.
// With one tile a wave needs ~220 registers, so eight waves (two per SIMD) fit a CU and
// keep twice the loads in flight that four do; more tiles need more than 256 registers
// per wave, one wave per SIMD, hence four.
template <int NT>
struct DecodeWaves {
  static constexpr int value = NT == 1 ? 8 : 4;
};

template <int NT, int W>
struct DecodeShared {
  float m[W][NT * 8];
  float l[W][NT * 8];
  float4 o[W][NT * 8][kD / 4];
  uint32_t last;
};

// Fused append: the group's own new rows are stored by the work item of its last
// chunk, which holds every block they fall in (the host makes sure of that), before its
// waves read them. Only the keys of this kv head.
template <int kThreads>
__device__ __forceinline__ void fused_append(const AttnItem& it, uint32_t kh, uint32_t hkv,
                                             uint32_t bpp_shift, const float* __restrict__ knew,
                                             const float* __restrict__ vnew,
                                             const uint32_t* __restrict__ kv_slot, _Float16* kw,
                                             _Float16* vw) {
  const uint32_t page_size = 16u << bpp_shift;
  for (uint32_t i = threadIdx.x; i < it.nrows * 32; i += kThreads) {
    const uint32_t row = it.r0 + i / 32, ch = (i / 2) % 16;
    const bool is_k = (i & 1) == 0;
    const float* src = (is_k ? knew : vnew) + (static_cast<size_t>(row) * hkv + kh) * kD + ch * 8;
    const uint32_t slot = kv_slot[row];
    const uint32_t off = slot & (page_size - 1);
    const size_t region = (static_cast<size_t>(slot >> (bpp_shift + 4)) * hkv + kh) * page_size * kD;
    _Float16* dst = is_k ? kw + region + k_offset(off, ch) : vw + region + off * kD + ch * 8;
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    *reinterpret_cast<half8*>(dst) =
        half8{static_cast<_Float16>(a.x), static_cast<_Float16>(a.y), static_cast<_Float16>(a.z),
              static_cast<_Float16>(a.w), static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
              static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
  }
  // Stores complete, then the workgroup barrier orders them before every wave's loads
  // (the waves of a workgroup share one CU and its L1).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Merges one group of a split-K pass (the last arrival does it): its chunk list is npre
// prefix chunks (slots from pre_base, logical rows from row_off * G on) followed by its
// own nown chunks (slots from own_base). A thread merges one (row, 4 dims) over a range
// of the list in list order, with a running maximum; the loads of 8 chunks are in
// flight at a time. With more than one round of loads (over 8 chunks) and threads to
// spare, the list is cut into `parts` contiguous ranges, each merged by its own
// nlog * 32 threads; part 0 then adds the others' results in part order through LDS (a
// fixed order, so the result does not depend on timing).
template <int kThreads, int kRows>
__device__ __forceinline__ void merge_group(uint32_t g_r0, uint32_t g_nrows, uint32_t own_base,
                                         uint32_t nown, uint32_t pre_base, uint32_t npre,
                                         uint32_t row_off, uint32_t kh, uint32_t G, uint32_t hq,
                                         uint32_t hkv, float* __restrict__ out,
                                         __amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rml) {
  __shared__ float4 part_o_lds[kThreads];
  __shared__ float2 part_ml_lds[kThreads];
  constexpr int kPer = (kRows * 32 + kThreads - 1) / kThreads;
  const size_t qd = static_cast<size_t>(hq) * kD;
  const uint32_t g_nlog = g_nrows * G, nall = npre + nown;
  auto entry = [&](uint32_t j, uint32_t lr) -> size_t {
    return j < npre ? ((static_cast<size_t>(pre_base) + j) * hkv + kh) * kRows + row_off * G + lr
                    : ((static_cast<size_t>(own_base) + (j - npre)) * hkv + kh) * kRows + lr;
  };
  auto merge_range = [&](uint32_t lr, uint32_t qi, uint32_t c_begin, uint32_t c_end, float& mt,
                         float& lt, float4& o) {
    for (uint32_t c0 = c_begin; c0 < c_end; c0 += 8) {
      float2 ml[8];
      float4 po[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const size_t e = entry(min(c0 + j, c_end - 1), lr);
        ml[j] = ld2_coherent(rml, static_cast<uint32_t>(e * 8));
        po[j] = ld4_coherent(ro, static_cast<uint32_t>((e * kD + qi * 4) * 4));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (c0 + j >= c_end || !(ml[j].y > 0.0f)) continue;  // past the range, or empty
        const float mn = fmaxf(mt, ml[j].x);
        const float r = __builtin_amdgcn_exp2f(mt - mn), wt = __builtin_amdgcn_exp2f(ml[j].x - mn);
        lt = lt * r + ml[j].y * wt;
        o.x = o.x * r + po[j].x * wt;
        o.y = o.y * r + po[j].y * wt;
        o.z = o.z * r + po[j].z * wt;
        o.w = o.w * r + po[j].w * wt;
        mt = mn;
      }
    }
  };
  auto store_row = [&](uint32_t lr, uint32_t qi, float lt, const float4& o) {
    const uint32_t rr = g_r0 + lr / G, h = kh * G + lr % G;
    const float inv = 1.0f / lt;
    *reinterpret_cast<float4*>(out + rr * qd + h * kD + qi * 4) = float4{o.x * inv, o.y * inv, o.z * inv, o.w * inv};
  };
  const uint32_t span = g_nlog * 32;
  const uint32_t parts = min(static_cast<uint32_t>(kThreads) / span, (nall + 7) / 8);  // uniform
  if (parts >= 2) {
    const uint32_t part = threadIdx.x / span, pi = threadIdx.x - part * span;
    const uint32_t lr = pi >> 5, qi = pi & 31;
    float mt = -INFINITY, lt = 0.0f;
    float4 o = {0, 0, 0, 0};
    if (part < parts) merge_range(lr, qi, nall * part / parts, nall * (part + 1) / parts, mt, lt, o);
    if (part > 0 && part < parts) {
      part_o_lds[threadIdx.x] = o;
      part_ml_lds[threadIdx.x] = float2{mt, lt};
    }
    __syncthreads();
    if (part == 0) {
      for (uint32_t pp = 1; pp < parts; ++pp) {
        const float2 b = part_ml_lds[pp * span + pi];
        if (!(b.y > 0.0f)) continue;
        const float4 ob = part_o_lds[pp * span + pi];
        const float mn = fmaxf(mt, b.x);
        const float r = __builtin_amdgcn_exp2f(mt - mn), wt = __builtin_amdgcn_exp2f(b.x - mn);
        lt = lt * r + b.y * wt;
        o = float4{o.x * r + ob.x * wt, o.y * r + ob.y * wt, o.z * r + ob.z * wt, o.w * r + ob.w * wt};
        mt = mn;
      }
      store_row(lr, qi, lt, o);
    }
    __syncthreads();  // the LDS results are read before another merge reuses them
    return;
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t idx = threadIdx.x + k * kThreads;
    const uint32_t lr = idx >> 5, qi = idx & 31;
    if (lr >= g_nlog || lr >= kRows) continue;
    float mt = -INFINITY, lt = 0.0f;
    float4 o = {0, 0, 0, 0};
    merge_range(lr, qi, 0, nall, mt, lt, o);
    store_row(lr, qi, lt, o);
  }
}

// Hands a workgroup's result for its logical rows on: straight to `out` when the item
// is its group's only chunk, else to the item's partial slot, after which the last item
// of the group to arrive merges all partials in chunk order (so the result does not
// depend on arrival order). value(lr, qi, mt, lt, o) gives the workgroup's maximum, sum
// and unnormalised O (dims 4qi..4qi+3) of logical row lr. With a shared prefix the
// group's chunk list is the prefix items' chunks, then its own; a prefix item arrives at
// every member group and merges each one it completes.
template <int kThreads, int kRows, bool kCascade = false, typename Value>
__device__ __forceinline__ void finish_item(const AttnItem& it, uint32_t kh, uint32_t G, uint32_t hq,
                                            uint32_t hkv, uint32_t nlog, float* __restrict__ out,
                                            float* __restrict__ part_o, float2* __restrict__ part_ml,
                                            uint32_t* __restrict__ counters, uint32_t part_o_bytes,
                                            uint32_t part_ml_bytes, uint32_t& last, Value value,
                                            const SubRef* __restrict__ members = nullptr) {
  const size_t qd = static_cast<size_t>(hq) * kD;
  const uint32_t rows_per_slot = kRows;
  const bool is_prefix = kCascade && (it.pref_info & kPrefixItem) != 0;
  const uint32_t total = it.nch + (kCascade && !is_prefix ? it.pref_nch : 0u);  // chunks of the group
  const bool direct = !is_prefix && total == 1;
  const size_t slot = (static_cast<size_t>(it.part_base) + it.chunk) * hkv + kh;
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(part_o, part_o_bytes);
  const __amdgpu_buffer_rsrc_t rml = make_rsrc(part_ml, part_ml_bytes);
  constexpr int kPer = (kRows * 32 + kThreads - 1) / kThreads;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t idx = threadIdx.x + k * kThreads;
    const uint32_t lr = idx >> 5, qi = idx & 31;
    if (lr >= nlog || lr >= kRows) continue;
    float mt, lt;
    float4 o;
    value(lr, qi, mt, lt, o);
    if (direct) {
      const uint32_t rr = it.r0 + lr / G, h = kh * G + lr % G;
      const float inv = 1.0f / lt;
      *reinterpret_cast<float4*>(out + rr * qd + h * kD + qi * 4) = float4{o.x * inv, o.y * inv, o.z * inv, o.w * inv};
    } else {
      const size_t e = slot * rows_per_slot + lr;
      st4_coherent(ro, static_cast<uint32_t>((e * kD + qi * 4) * 4), o);
      if (qi == 0) st2_coherent(rml, static_cast<uint32_t>(e * 8), float2{mt, lt});
    }
  }
  if (direct) return;

  // Arrival: at the item's own group, or (prefix item) at every member group; a group's
  // last arrival merges it.
  // Memory order. Every access to a partial is device-coherent at the instruction: the
  // stores write through (sc1) to the memory all XCDs share, the merge loads (sc1) read
  // from it and never from a possibly stale L2 line; these are the instructions the
  // gfx942/gfx950 memory model uses for agent-scope atomic stores and loads. What is
  // left is the order between those accesses and the counter:
  //  - producer: s_waitcnt(0) waits until every store of this thread is acknowledged
  //    by the coherence point (a write-through store is acknowledged only when it is
  //    there), and the workgroup barrier makes thread 0's increment wait for every
  //    thread's wait; so the increment is issued after all partials are in memory;
  //  - consumer: the merge loads are issued after the barrier that follows thread 0's
  //    increment, whose result (control dependency) decides whether they run at all, so
  //    no merge load is issued before the counter has counted every producer.
  // A release increment and an acquire fence would add an L2 write-back (buffer_wbl2)
  // and an L2 invalidate (buffer_inv) on every arrival, which this data does not need:
  // measured at the headline, 25.7 -> 27.6 us per launch (release alone +1.0 us,
  // acquire alone +0.35 us).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if constexpr (kCascade) {
    if (is_prefix) {
      __shared__ uint32_t done[16];  // the member groups this item completes
      const uint32_t nm = it.pref_nch;
      if (threadIdx.x < nm) {
        const SubRef& sr = members[it.pref_base + threadIdx.x];
        uint32_t* cnt = counters + (static_cast<size_t>(sr.counter) * hkv + kh) * kCounterStride;
        const uint32_t arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool fin = arrived == sr.nch + it.nch - 1;
        if (fin) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        done[threadIdx.x] = fin;
      }
      __syncthreads();
      for (uint32_t m = 0; m < nm; ++m) {
        if (!done[m]) continue;  // uniform (LDS)
        const SubRef sr = members[it.pref_base + m];
        merge_group<kThreads, kRows>(sr.r0, sr.nrows, sr.part_base, sr.nch, it.part_base, it.nch,
                                     sr.row_off, kh, G, hq, hkv, out, ro, rml);
      }
      return;
    }
  }
  if (threadIdx.x == 0) {
    uint32_t* cnt = counters + (static_cast<size_t>(it.counter) * hkv + kh) * kCounterStride;
    const uint32_t arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = arrived == total - 1;
    if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();

  if (!last) return;
  merge_group<kThreads, kRows>(it.r0, it.nrows, it.part_base, it.nch,
                               kCascade ? it.pref_base : 0u, kCascade ? it.pref_nch : 0u,
                               kCascade ? it.pref_info : 0u, kh, G, hq, hkv, out, ro, rml);
}

template <int NT, int kWaves = DecodeWaves<NT>::value>
__global__ __launch_bounds__(64 * kWaves) void paged_attn_decode(
    const AttnItem* __restrict__ items, const uint32_t* __restrict__ pos,
    const uint32_t* __restrict__ pages, const _Float16* kc, const _Float16* vc,
    const float* __restrict__ q, float* __restrict__ out,
    float* __restrict__ part_o, float2* __restrict__ part_ml, uint32_t* __restrict__ counters,
    const float* __restrict__ knew, const float* __restrict__ vnew,
    const uint32_t* __restrict__ kv_slot, _Float16* kw, _Float16* vw,  // kw/vw alias kc/vc
    uint32_t part_o_bytes, uint32_t part_ml_bytes, uint32_t hq, uint32_t hkv,
    uint32_t bpp_shift, uint32_t window, float scale_log2) {
  __shared__ DecodeShared<NT, kWaves> sh;
  const AttnItem it = items[blockIdx.x];
  const uint32_t kh = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  const bool lo_half = c >= 8;
  const uint32_t G = hq / hkv;
  const uint32_t nlog = it.nrows * G;  // logical rows in the group

  if (knew != nullptr && it.chunk == it.nch - 1 && !(it.pref_info & kPrefixItem))
    fused_append<64 * kWaves>(it, kh, hkv, bpp_shift, knew, vnew, kv_slot, kw, vw);

  // This wave's share of the item's blocks, [wb0, wb1), in whole quads of blocks (a
  // static split: the result does not depend on timing); at most 64 blocks per wave,
  // one page id per lane.
  const uint32_t nall = it.blk1 - it.blk0;
  const uint32_t quads = (nall + 3) / 4;
  const uint32_t wb0 = it.blk0 + 4 * (quads * wave / kWaves);
  const uint32_t wb1 = min(it.blk1, it.blk0 + 4 * (quads * (wave + 1) / kWaves));
  const uint32_t nblk = wb1 > wb0 ? wb1 - wb0 : 0;
  const uint32_t bpp_mask = (1u << bpp_shift) - 1u;  // blocks per page - 1
  const size_t head_stride = static_cast<size_t>(16u << bpp_shift) * kD;  // halves per (page, head)
  const uint32_t* pt = pages + it.pt_off;
  int pid = 0;  // page id of block wb0 + lane
  if (static_cast<uint32_t>(lane) < nblk) pid = static_cast<int>(pt[(wb0 + lane) >> bpp_shift]);
  auto block_off = [&](uint32_t b) -> size_t {  // b relative to wb0, clamped to [wb0, wb1)
    b = b < nblk ? b : nblk - 1;
    const uint32_t page = static_cast<uint32_t>(__builtin_amdgcn_readlane(pid, static_cast<int>(b)));
    return (static_cast<size_t>(page) * hkv + kh) * head_stride +
           static_cast<size_t>((wb0 + b) & bpp_mask) * 16 * kD;
  };
  const int key_end = static_cast<int>(wb1 * 16);

  // Two register sets of two blocks each, used in turn: the loads of one set are in
  // flight while the other is computed.
  BlockRegs s0[2], s1[2];
  auto load_pair = [&](BlockRegs* r, uint32_t b) {
    const size_t o0 = block_off(b), o1 = block_off(b + 1);
    load_block(r[0], kc + o0, vc + o0, lane);
    load_block(r[1], kc + o1, vc + o1, lane);
    // Keep the loads here: the scheduler would otherwise sink them below the compute
    // of the other set, leaving nothing in flight while it runs.
    __builtin_amdgcn_sched_barrier(0);
  };
  if (nblk > 0) load_pair(s0, 0);  // first, so HBM is busy while q is set up

  // Per tile: this lane's column's row position and key window, and the q operand.
  half8 qb[NT][4];
  int rpos[NT], rlo[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint32_t lr = t * 8 + (c & 7);
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
          const _Float16 hi = static_cast<_Float16>(x[e]);
          qb[t][pp][e] = lo_half ? static_cast<_Float16>(x[e] - static_cast<float>(hi)) : hi;
        }
      }
    } else {
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) qb[t][pp] = half8{0, 0, 0, 0, 0, 0, 0, 0};
    }
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

  auto process_pair = [&](const BlockRegs* r, uint32_t b) {
    const int kb0 = static_cast<int>((wb0 + b) * 16) + 4 * g;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float x[8];
      float bmax = -INFINITY;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        floatx4 sc = {0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < 4; ++p) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r[h].k[p], qb[t][p], sc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float full = sc[i] + xor8(sc[i]);
          const int kp = kb0 + h * 16 + i;
          const bool ok = (kp >= rlo[t]) & (kp <= rpos[t]) & (kp < key_end);  // no branches
          x[h * 4 + i] = ok ? full * scale_log2 : -INFINITY;
          bmax = fmaxf(bmax, x[h * 4 + i]);
        }
      }
      bmax = max_xor32(max_xor16(bmax));
      const float mn = fmaxf(m[t], bmax);
      const bool live = mn != -INFINITY;
      float pr[8], rs = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pr[i] = live ? __builtin_amdgcn_exp2f(x[i] - mn) : 0.0f;
        rs += pr[i];
      }
      rs = sum_xor32(sum_xor16(rs));
      // Rescale only when some column's maximum moved (wave-uniform test).
      if (__builtin_amdgcn_ballot_w64(mn != m[t])) {
        const float corr = live ? __builtin_amdgcn_exp2f(m[t] - mn) : 1.0f;
        l[t] *= corr;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[t][j] *= corr;
      }
      l[t] += rs;
      m[t] = mn;
      // PV over both blocks at once (16x16x32): element e of the P operand is key
      // (e / 4) * 16 + 4g + e % 4 of the pair, as in the V operand.
      half8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 hi = static_cast<_Float16>(pr[e]);
        pb[e] = lo_half ? static_cast<_Float16>(pr[e] - static_cast<float>(hi)) : hi;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const half8 a = {r[0].v[0][j], r[0].v[1][j], r[0].v[2][j], r[0].v[3][j],
                         r[1].v[0][j], r[1].v[1][j], r[1].v[2][j], r[1].v[3][j]};
        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, acc[t][j], 0, 0, 0);
      }
    }
  };

  if (nblk > 0) {
    // In the loop, loads and compute are unconditional: a conditional use would let the
    // compiler sink the prefetch into it, and every path keeps the same loads in flight
    // so the waits before each use stay partial. The last quad is peeled so that no
    // load is issued past the end.
    uint32_t b = 0;
    for (; b + 4 < nblk; b += 4) {
      load_pair(s1, b + 2);
      process_pair(s0, b);
      load_pair(s0, b + 4);
      process_pair(s1, b + 2);
    }
    if (b + 2 < nblk) {
      load_pair(s1, b + 2);
      process_pair(s0, b);
      process_pair(s1, b + 2);
    } else {
      process_pair(s0, b);
    }
  }

  // Join the hi and lo columns (lanes c and c^8 hold the same logical row), then hand
  // each wave's (m, l, O) of its logical rows to LDS.
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][j][i] += xor8(acc[t][j][i]);
    const int lr = t * 8 + c;
    if (c < 8) {
      if (g == 0) {
        sh.m[wave][lr] = m[t];
        sh.l[wave][lr] = l[t];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sh.o[wave][lr][g * 8 + i * 2] = float4{acc[t][0][i], acc[t][1][i], acc[t][2][i], acc[t][3][i]};
        sh.o[wave][lr][g * 8 + i * 2 + 1] = float4{acc[t][4][i], acc[t][5][i], acc[t][6][i], acc[t][7][i]};
      }
    }
  }
  __syncthreads();

  // Merge the waves: thread -> (row, 4 dims); NT*8 rows x 32 quads = NT * 256 values.
  finish_item<64 * kWaves, NT * 8>(it, kh, G, hq, hkv, nlog, out, part_o, part_ml, counters,
                                   part_o_bytes, part_ml_bytes, sh.last,
                                   [&](uint32_t lr, uint32_t qi, float& mt, float& lt, float4& o) {
    mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mt = fmaxf(mt, sh.m[w][lr]);
    lt = 0.0f;
    o = float4{0, 0, 0, 0};
    if (mt != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = __builtin_amdgcn_exp2f(sh.m[w][lr] - mt);  // 0 for an empty wave
        lt += sh.l[w][lr] * wt;
        const float4 ow = sh.o[w][lr][qi];
        o.x += ow.x * wt;
        o.y += ow.y * wt;
        o.z += ow.z * wt;
        o.w += ow.w * wt;
      }
    }
  });
}


// Balanced one-tile decode: the waves of a workgroup take the item's quads of blocks
// from a queue in LDS as they finish the previous one, so a wave whose loads come back
// late takes fewer quads instead of holding up the workgroup. Each quad's softmax state
// starts afresh and goes to its own LDS slot, and the slots are merged in quad order,
// so the result does not depend on which wave ran which quad. At most kBalQuads quads
// (64 blocks) per item; block loads go through buffer resources whose size is zero for
// blocks past the item's end, so the prefetch of a quad that does not exist reads
// nothing. A wave keeps two blocks (16 KiB) in flight: measured against two pairs, as
// fast or faster, with fewer registers.
static constexpr int kBalWaves = 8;
static constexpr uint32_t kBalQuads = 16;
static constexpr int kNontemporal = 2;  // nt

struct BalancedShared {
  float m[kBalQuads][8];
  float l[kBalQuads][8];
  float4 o[kBalQuads][8][kD / 4];
  float q[8][kD];            // the item's queries when the kernel normalises and rotates them
  float qsq[kBalWaves][kD];  // per-wave scratch of that step
  uint32_t next;
  uint32_t last;
};

// kPolicy: the loads' cache policy (nontemporal for K/V read once; the default, which
// keeps the lines in L2, for blocks that other work items read too).
template <int kPolicy = kNontemporal>
__device__ __forceinline__ void load_block_buf(BlockRegs& r, const _Float16* kblk, const _Float16* vblk,
                                               bool valid, int lane) {
  const int c = lane & 15, g = lane >> 4;
  const int bytes = valid ? 2048 * 2 : 0;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(kblk), 0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(vblk), 0, bytes, 0x00020000);
#pragma unroll
  for (int p = 0; p < 4; ++p)  // [p][key c][g] in 16-byte units
    r.k[p] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, ((c * 4 + g) + p * 64) * 16, 0, kPolicy));
#pragma unroll
  for (int i = 0; i < 4; ++i)  // key 4g + i, dims c*8..c*8+7
    r.v[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rv, ((4 * g + i) * kD + c * 8) * 2, 0, kPolicy));
}

// The inputs of write_rows when the kernel runs it itself (Backend::attention in one
// launch): the rows' projected qkv, the norm weights and the layer's RoPE table.
struct QkvIn {
  const float* qkv;
  const float* q_norm;
  const float* k_norm;
  const float* rope_cs;
  uint32_t rope_len;
  float eps;
};

// write_rows inside the attention kernel: wave t normalises and rotates logical row t's
// query head into q_lds[t] (write_rows' arithmetic, the same bits), then (item of the
// group's last chunk only) row t - nlog's key head, which it stores with the row's
// value head. Ends with a workgroup barrier after the stores have completed, which
// orders them and the queries in LDS before every wave's reads.
template <int kWaves>
__device__ __forceinline__ void fused_write_rows(const AttnItem& it, uint32_t kh, uint32_t G,
                                                 uint32_t hq, uint32_t hkv, uint32_t nlog,
                                                 uint32_t bpp_shift, const uint32_t* pos,
                                                 const uint32_t* __restrict__ kv_slot,
                                                 const QkvIn& qi_in, float (*q_lds)[kD],
                                                 float* qsq, int wave, int lane, _Float16* kw,
                                                 _Float16* vw) {
  const uint32_t nk = (it.chunk == it.nch - 1 && !(it.pref_info & kPrefixItem)) ? it.nrows : 0;
  const uint32_t qd = hq * kD, kvd = hkv * kD, cols = qd + 2 * kvd;
  for (uint32_t t = static_cast<uint32_t>(wave); t < nlog + nk; t += kWaves) {
    float o0, o1;
    if (t < nlog) {
      const uint32_t rr = it.r0 + t / G, h = kh * G + t % G;
      norm_rope_head(qi_in.qkv + static_cast<size_t>(rr) * cols + h * kD, qi_in.q_norm,
                     qi_in.rope_cs, qi_in.rope_len, pos[rr], qi_in.eps, lane, qsq, o0, o1);
      q_lds[t][lane] = o0;
      q_lds[t][lane + 64] = o1;
    } else {
      const uint32_t rr = it.r0 + (t - nlog);
      const float* ks = qi_in.qkv + static_cast<size_t>(rr) * cols + qd + kh * kD;
      norm_rope_head(ks, qi_in.k_norm, qi_in.rope_cs, qi_in.rope_len, pos[rr], qi_in.eps, lane,
                     qsq, o0, o1);
      store_kv_head(o0, o1, ks + kvd, kv_slot[rr], kh, hkv, bpp_shift + 4, lane, kw, vw);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// QKV: instead of reading q (and storing knew/vnew), the workgroup normalises and rotates
// its rows' q heads from qkv into LDS (write_rows' arithmetic, the same bits), and the
// item of the group's last chunk normalises, rotates and stores the rows' key heads and
// stores their value heads, before any wave reads a block.
// UB: blocks per queue unit (4, or 2 for items of at most 32 blocks, so that every wave
// has a unit).
template <bool QKV, int UB>
__global__ __launch_bounds__(64 * kBalWaves) void paged_attn_decode_balanced(
    const AttnItem* __restrict__ items, const uint32_t* pos,
    const uint32_t* __restrict__ pages, const _Float16* kc, const _Float16* vc,
    const float* q, float* __restrict__ out,
    float* __restrict__ part_o, float2* __restrict__ part_ml, uint32_t* __restrict__ counters,
    const float* __restrict__ knew, const float* __restrict__ vnew,
    const uint32_t* __restrict__ kv_slot, _Float16* kw, _Float16* vw,  // kw/vw alias kc/vc
    uint32_t part_o_bytes, uint32_t part_ml_bytes, uint32_t hq, uint32_t hkv,
    uint32_t bpp_shift, uint32_t window, float scale_log2, QkvIn qi_in) {
  __shared__ BalancedShared sh;
  const AttnItem it = items[blockIdx.x];
  const uint32_t kh = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  const bool lo_half = c >= 8;
  const uint32_t G = hq / hkv;
  const uint32_t nlog = it.nrows * G;  // logical rows in the group (at most 8)

  if (threadIdx.x == 0) sh.next = kBalWaves;  // quads 0..W-1 go to waves 0..W-1
  if constexpr (QKV) {
    fused_write_rows<kBalWaves>(it, kh, G, hq, hkv, nlog, bpp_shift, pos, kv_slot, qi_in, sh.q,
                                sh.qsq[wave], wave, lane, kw, vw);
  } else if (knew != nullptr && it.chunk == it.nch - 1 && !(it.pref_info & kPrefixItem)) {
    fused_append<64 * kBalWaves>(it, kh, hkv, bpp_shift, knew, vnew, kv_slot, kw, vw);
  } else {
    __syncthreads();
  }

  const uint32_t nall = it.blk1 - it.blk0;  // at most UB * kBalQuads (host-checked)
  const uint32_t nq = (nall + UB - 1) / UB;  // queue units
  const uint32_t bpp_mask = (1u << bpp_shift) - 1u;
  const size_t head_stride = static_cast<size_t>(16u << bpp_shift) * kD;
  const uint32_t* pt = pages + it.pt_off;
  int pid = 0;  // page id of block blk0 + lane
  if (static_cast<uint32_t>(lane) < nall) pid = static_cast<int>(pt[(it.blk0 + lane) >> bpp_shift]);
  const int key_end = static_cast<int>(it.blk1 * 16);

  // Two register sets of one block each, used in turn: the loads of one are in flight
  // while the other is computed.
  BlockRegs s0, s1;
  // Loads block b (relative to blk0; wave-uniform) into r.
  auto load_set = [&](BlockRegs& r, uint32_t b) {
    const bool valid = b < nall;
    const uint32_t page = static_cast<uint32_t>(__builtin_amdgcn_readlane(pid, static_cast<int>(valid ? b : 0)));
    const size_t o = (static_cast<size_t>(page) * hkv + kh) * head_stride +
                     static_cast<size_t>((it.blk0 + b) & bpp_mask) * 16 * kD;
    load_block_buf(r, kc + o, vc + o, valid, lane);
    __builtin_amdgcn_sched_barrier(0);
  };
  // This lane's column: its row's position and key window; q is read before the first
  // blocks (so that waiting for it does not wait for them) and split into the hi or lo
  // part after.
  // (Unconditional loads, clamped to a valid row: a branch around them would make the
  // compiler wait for every load before the first block's page id.)
  const bool has_row = (c & 7) < nlog;
  const uint32_t lr0 = has_row ? (c & 7) : 0;
  const uint32_t rr0 = it.r0 + lr0 / G, h0 = kh * G + lr0 % G;
  const int p0 = static_cast<int>(pos[rr0]);
  const int rpos = has_row ? p0 : -1;
  const int rlo = (window > 0 && p0 + 1 > static_cast<int>(window)) ? p0 + 1 - static_cast<int>(window) : 0;
  float4 qraw[8];
  {
    const float* qp = QKV ? &sh.q[lr0][g * 8] : q + (static_cast<size_t>(rr0) * hq + h0) * kD + g * 8;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      qraw[2 * pp] = *reinterpret_cast<const float4*>(qp + pp * 32);
      qraw[2 * pp + 1] = *reinterpret_cast<const float4*>(qp + pp * 32 + 4);
    }
  }
  // Issue them here, ahead of the blocks (q and pos are not declared __restrict__ and the
  // empty asm may write memory, so the compiler cannot sink the loads to their use; the
  // scheduling barrier keeps the scheduler from doing so).
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  uint32_t qc = static_cast<uint32_t>(wave);  // this wave's current quad
  load_set(s0, UB * qc);
  load_set(s1, UB * qc + 1);
  half8 qb[4];
#pragma unroll
  for (int pp = 0; pp < 4; ++pp) {
    const float4 a = qraw[2 * pp], b = qraw[2 * pp + 1];
    float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = has_row ? x[e] : 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 hi = static_cast<_Float16>(x[e]);
      qb[pp][e] = lo_half ? static_cast<_Float16>(x[e] - static_cast<float>(hi)) : hi;
    }
  }

  float m, l;
  floatx4 acc[8];
  auto process_set = [&](const BlockRegs& r, uint32_t b) {
    const int kb0 = static_cast<int>((it.blk0 + b) * 16) + 4 * g;
    float x[4];
    float bmax = -INFINITY;
    floatx4 sc = {0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < 4; ++p) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.k[p], qb[p], sc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float full = sc[i] + xor8(sc[i]);
      const int kp = kb0 + i;
      const bool ok = (kp >= rlo) & (kp <= rpos) & (kp < key_end);
      x[i] = ok ? full * scale_log2 : -INFINITY;
      bmax = fmaxf(bmax, x[i]);
    }
    bmax = max_xor32(max_xor16(bmax));
    const float mn = fmaxf(m, bmax);
    const bool live = mn != -INFINITY;
    float pr[4], rs = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = live ? __builtin_amdgcn_exp2f(x[i] - mn) : 0.0f;
      rs += pr[i];
    }
    rs = sum_xor32(sum_xor16(rs));
    if (__builtin_amdgcn_ballot_w64(mn != m)) {
      const float corr = live ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
      l *= corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= corr;
    }
    l += rs;
    m = mn;
    // PV (16x16x16): element e of the P operand is key 4g + e, as in the V operand.
    half4 pb;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const _Float16 hi = static_cast<_Float16>(pr[e]);
      pb[e] = lo_half ? static_cast<_Float16>(pr[e] - static_cast<float>(hi)) : hi;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const half4 a = {r.v[0][j], r.v[1][j], r.v[2][j], r.v[3][j]};
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb, acc[j], 0, 0, 0);
    }
  };

  while (qc < nq) {
    uint32_t taken = 0;
    if (lane == 0) taken = __hip_atomic_fetch_add(&sh.next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const uint32_t qn = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(taken)));
    m = -INFINITY;
    l = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = floatx4{0, 0, 0, 0};
    // The unit's blocks in turn; each load goes two blocks ahead, into the next unit
    // for the last two.
    static_assert(UB == 2 || UB == 4, "units of two or four blocks");
#pragma unroll
    for (uint32_t j = 0; j < UB; ++j) {
      BlockRegs& set = (j & 1) ? s1 : s0;
      process_set(set, UB * qc + j);
      load_set(set, j + 2 < UB ? UB * qc + j + 2 : UB * qn + (j + 2 - UB));
    }
    // Join the hi and lo columns and store the quad's state in its slot.
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][i] += xor8(acc[j][i]);
    if (c < 8) {
      if (g == 0) {
        sh.m[qc][c] = m;
        sh.l[qc][c] = l;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sh.o[qc][c][g * 8 + i * 2] = float4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
        sh.o[qc][c][g * 8 + i * 2 + 1] = float4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]};
      }
    }
    qc = qn;
  }
  __syncthreads();

  finish_item<64 * kBalWaves, 8>(it, kh, G, hq, hkv, nlog, out, part_o, part_ml, counters,
                                 part_o_bytes, part_ml_bytes, sh.last,
                                 [&](uint32_t lr, uint32_t qi, float& mt, float& lt, float4& o) {
    mt = -INFINITY;
    for (uint32_t k = 0; k < nq; ++k) mt = fmaxf(mt, sh.m[k][lr]);
    lt = 0.0f;
    o = float4{0, 0, 0, 0};
    if (mt == -INFINITY) return;
    for (uint32_t k = 0; k < nq; ++k) {
      const float wt = __builtin_amdgcn_exp2f(sh.m[k][lr] - mt);  // 0 for an empty quad
      lt += sh.l[k][lr] * wt;
      const float4 ow = sh.o[k][lr][qi];
      o.x += ow.x * wt;
      o.y += ow.y * wt;
      o.z += ow.z * wt;
      o.w += ow.w * wt;
    }
  });
}

// 16-row-tile decode (NT = 1 or 2 tiles of 16 logical rows): the kernel for passes of
// more than 8 logical rows per work item (verify), and for one-tile passes whose work
// items split evenly over its waves or are longer than the queue kernel takes. Each
// logical row is one MFMA column: q's f16 hi and lo parts are two B operands whose
// products accumulate into the same S (and P's into the same O), instead of taking two
// columns per row as in the 8-row tiles: the same MFMA work per logical row, half the
// softmax arithmetic (no column is duplicated), and, with one-block register sets, a
// wave fits 256 registers, so two waves run per SIMD. The item's blocks are split over
// the waves evenly, to a block (a static split: the result does not depend on timing).
static constexpr int kWideWaves = 8;

template <int NT, bool QKV>
struct WideShared {
  float m[kWideWaves][NT * 16];
  float l[kWideWaves][NT * 16];
  float4 o[kWideWaves][NT * 16][kD / 4];
  uint32_t last;
};
// QKV: as in the queue kernel, the workgroup runs write_rows for its rows first
// (queries into LDS, the last chunk's item stores the rows' K/V). The queries and the
// sum-of-squares scratch borrow the space of the waves' partial results, which is
// written only after every wave has taken its queries into registers.
// CASC: the pass has shared-prefix items, whose blocks other prefix items read as well:
// those load with the default cache policy (kept in L2) instead of nontemporal (cfg2:
// 19.0 -> 17.5 us). A separate instantiation, since the per-item choice costs the
// passes without shared prefixes 0.7-1.7 us.
template <int NT, bool QKV, bool CASC = false>
__global__ __launch_bounds__(64 * kWideWaves) void paged_attn_decode_wide(
    const AttnItem* __restrict__ items, const uint32_t* pos,
    const uint32_t* __restrict__ pages, const _Float16* kc, const _Float16* vc,
    const float* q, float* __restrict__ out,
    float* __restrict__ part_o, float2* __restrict__ part_ml, uint32_t* __restrict__ counters,
    const float* __restrict__ knew, const float* __restrict__ vnew,
    const uint32_t* __restrict__ kv_slot, _Float16* kw, _Float16* vw,  // kw/vw alias kc/vc
    uint32_t part_o_bytes, uint32_t part_ml_bytes, uint32_t hq, uint32_t hkv,
    uint32_t bpp_shift, uint32_t window, float scale_log2, QkvIn qi_in,
    const SubRef* __restrict__ members) {
  __shared__ WideShared<NT, false> sh;
  static_assert(sizeof(sh.o) >= (NT * 16 + kWideWaves) * kD * sizeof(float), "q and scratch fit");
  float (*const q_lds)[kD] = reinterpret_cast<float (*)[kD]>(&sh.o[0][0][0]);
  float* const qsq_lds = reinterpret_cast<float*>(&sh.o[0][0][0]) + NT * 16 * kD;
  const AttnItem it = items[blockIdx.x];
  const uint32_t kh = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  const uint32_t G = hq / hkv;
  const uint32_t nlog = it.nrows * G;  // logical rows in the group (at most NT * 16)

  if constexpr (QKV)
    fused_write_rows<kWideWaves>(it, kh, G, hq, hkv, nlog, bpp_shift, pos, kv_slot, qi_in, q_lds,
                                 qsq_lds + wave * kD, wave, lane, kw, vw);
  else if (knew != nullptr && it.chunk == it.nch - 1 && !(it.pref_info & kPrefixItem))
    fused_append<64 * kWideWaves>(it, kh, hkv, bpp_shift, knew, vnew, kv_slot, kw, vw);

  // This wave's share of the item's blocks, [wb0, wb1): shares differ by at most one
  // block; at most 64 blocks per wave, one page id per lane.
  const uint32_t nall = it.blk1 - it.blk0;
  const uint32_t wb0 = it.blk0 + nall * wave / kWideWaves;
  const uint32_t wb1 = it.blk0 + nall * (wave + 1) / kWideWaves;
  const uint32_t nblk = wb1 - wb0;
  const uint32_t bpp_mask = (1u << bpp_shift) - 1u;
  const size_t head_stride = static_cast<size_t>(16u << bpp_shift) * kD;
  const uint32_t* pt = pages + it.pt_off;
  int pid = 0;  // page id of block wb0 + lane
  if (static_cast<uint32_t>(lane) < nblk) pid = static_cast<int>(pt[(wb0 + lane) >> bpp_shift]);
  const int key_end = static_cast<int>(wb1 * 16);
  const bool shared_blocks = (it.pref_info & kPrefixItem) != 0;

  BlockRegs s0, s1;
  // Loads block b (relative to wb0; wave-uniform) into r; past nblk it reads nothing.
  auto load_set = [&](BlockRegs& r, uint32_t b) {
    const bool valid = b < nblk;
    const uint32_t page = static_cast<uint32_t>(__builtin_amdgcn_readlane(pid, static_cast<int>(valid ? b : 0)));
    const size_t o = (static_cast<size_t>(page) * hkv + kh) * head_stride +
                     static_cast<size_t>((wb0 + b) & bpp_mask) * 16 * kD;
    if constexpr (CASC) {
      if (shared_blocks)  // uniform: a shared prefix, read by the other prefix groups too
        load_block_buf<0>(r, kc + o, vc + o, valid, lane);
      else
        load_block_buf(r, kc + o, vc + o, valid, lane);
    } else {
      load_block_buf(r, kc + o, vc + o, valid, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Per tile: this lane's column's row position and key window, and q (clamped to a
  // valid row, zeroed after the load for columns past the group's rows).
  int rpos[NT], rlo[NT];
  float4 qraw[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint32_t lr = t * 16 + c;
    const uint32_t lrc = lr < nlog ? lr : 0;
    const uint32_t rr = it.r0 + lrc / G, h = kh * G + lrc % G;
    const int p = static_cast<int>(pos[rr]);
    rpos[t] = lr < nlog ? p : -1;
    rlo[t] = (window > 0 && p + 1 > static_cast<int>(window)) ? p + 1 - static_cast<int>(window) : 0;
    const float* qp;
    if constexpr (QKV) qp = &q_lds[lrc][g * 8];
    else qp = q + (static_cast<size_t>(rr) * hq + h) * kD + g * 8;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      qraw[t][2 * pp] = *reinterpret_cast<const float4*>(qp + pp * 32);
      qraw[t][2 * pp + 1] = *reinterpret_cast<const float4*>(qp + pp * 32 + 4);
    }
  }
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  load_set(s0, 0);
  load_set(s1, 1);
  half8 qh[NT][4], ql[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const bool has_row = static_cast<uint32_t>(t * 16 + c) < nlog;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const float4 a = qraw[t][2 * pp], b = qraw[t][2 * pp + 1];
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = has_row ? x[e] : 0.0f;
        const _Float16 hi = static_cast<_Float16>(v);
        qh[t][pp][e] = hi;
        ql[t][pp][e] = static_cast<_Float16>(v - static_cast<float>(hi));
      }
    }
  }
  // Every wave holds its queries before any wave writes its partial result over them.
  if constexpr (QKV) __syncthreads();

  float m[NT], l[NT];
  floatx4 acc[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m[t] = -INFINITY;
    l[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[t][j] = floatx4{0, 0, 0, 0};
  }

  auto process_set = [&](const BlockRegs& r, uint32_t b) {
    const int kb0 = static_cast<int>((wb0 + b) * 16) + 4 * g;
    half4 va[8];  // V^T operand: dims c*8 + j of keys 4g..4g+3
#pragma unroll
    for (int j = 0; j < 8; ++j) va[j] = half4{r.v[0][j], r.v[1][j], r.v[2][j], r.v[3][j]};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      floatx4 sh_ = {0, 0, 0, 0}, sl_ = {0, 0, 0, 0};
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        sh_ = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.k[p], qh[t][p], sh_, 0, 0, 0);
        sl_ = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.k[p], ql[t][p], sl_, 0, 0, 0);
      }
      float x[4];
      float bmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kp = kb0 + i;
        const bool ok = (kp >= rlo[t]) & (kp <= rpos[t]) & (kp < key_end);
        x[i] = ok ? (sh_[i] + sl_[i]) * scale_log2 : -INFINITY;
        bmax = fmaxf(bmax, x[i]);
      }
      bmax = max_xor32(max_xor16(bmax));
      const float mn = fmaxf(m[t], bmax);
      const bool live = mn != -INFINITY;
      float pr[4], rs = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = live ? __builtin_amdgcn_exp2f(x[i] - mn) : 0.0f;
        rs += pr[i];
      }
      rs = sum_xor32(sum_xor16(rs));
      if (__builtin_amdgcn_ballot_w64(mn != m[t])) {
        const float corr = live ? __builtin_amdgcn_exp2f(m[t] - mn) : 1.0f;
        l[t] *= corr;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[t][j] *= corr;
      }
      l[t] += rs;
      m[t] = mn;
      half4 ph, pl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 hi = static_cast<_Float16>(pr[e]);
        ph[e] = hi;
        pl[e] = static_cast<_Float16>(pr[e] - static_cast<float>(hi));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va[j], ph, acc[t][j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va[j], pl, acc[t][j], 0, 0, 0);
    }
  };

  // Pairs of blocks, loads and compute unconditional (a block past nblk reads nothing
  // and is masked); each load goes two blocks ahead.
  for (uint32_t b = 0; b < nblk; b += 2) {
    process_set(s0, b);
    load_set(s0, b + 2);
    process_set(s1, b + 1);
    load_set(s1, b + 3);
  }

  // Each wave's (m, l, O) of its logical rows to LDS; O dims 32g + 8i + j per lane (the
  // group's rows only: the merge reads no other; headline 25.87 -> 25.74 us).
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int lr = t * 16 + c;
    if (g == 0) {
      sh.m[wave][lr] = m[t];
      sh.l[wave][lr] = l[t];
    }
    if (static_cast<uint32_t>(lr) < nlog)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sh.o[wave][lr][g * 8 + i * 2] = float4{acc[t][0][i], acc[t][1][i], acc[t][2][i], acc[t][3][i]};
      sh.o[wave][lr][g * 8 + i * 2 + 1] = float4{acc[t][4][i], acc[t][5][i], acc[t][6][i], acc[t][7][i]};
    }
  }
  __syncthreads();

  finish_item<64 * kWideWaves, NT * 16, true>(it, kh, G, hq, hkv, nlog, out, part_o, part_ml, counters,
                                        part_o_bytes, part_ml_bytes, sh.last,
                                        [&](uint32_t lr, uint32_t qi, float& mt, float& lt, float4& o) {
    mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWideWaves; ++w) mt = fmaxf(mt, sh.m[w][lr]);
    lt = 0.0f;
    o = float4{0, 0, 0, 0};
    if (mt == -INFINITY) return;
#pragma unroll
    for (int w = 0; w < kWideWaves; ++w) {
      const float wt = __builtin_amdgcn_exp2f(sh.m[w][lr] - mt);  // 0 for an empty wave
      lt += sh.l[w][lr] * wt;
      const float4 ow = sh.o[w][lr][qi];
      o.x += ow.x * wt;
      o.y += ow.y * wt;
      o.z += ow.z * wt;
      o.w += ow.w * wt;
    }
  }, members);
}

// ---------------------------------------------------------------------------------
// f32 arena (the reference's own K/V precision): K and V both `[page][kv_head]
// [page_size][128]` f32. Same structure as the 16-row-tile kernel (16 logical rows, one
// per MFMA column; static split of blocks over 8 waves; partials through LDS; split-K
// hand-off), with v_mfma_f32_16x16x4_f32: exact f32 products, f32 accumulation, no
// hi/lo split. Operand layouts (lane l, c = l % 16, g = l / 16), chosen so that every
// load instruction reads whole 64-byte pieces of key rows:
//   QK, step s = 4j + e (32 steps): lane holds K[key c][16j + 4g + e] and
//     q[row c][16j + 4g + e]; S^T[key 4g + i][col c] lands in element i of the four
//     partial sums (steps s % 4). Load j: 64 contiguous bytes of each of the 16 keys.
//   PV, step (t, m): lane holds V[key 4g + t][dim 64(m / 4) + 4c + m % 4] (A) and
//     P[key 4g + t][col c] (B); the output lands as dims 64h + 16g + 4i + (0..3) of
//     column c for h = 0, 1. Load (t, h): 256 contiguous bytes of each of 4 keys.
struct BlockRegsF32 {
  float4 k[8];
  float4 v[8];
};

__device__ __forceinline__ void load_block_f32(BlockRegsF32& r, const float* kblk, const float* vblk,
                                               bool valid, int lane) {
  const int c = lane & 15, g = lane >> 4;
  const int bytes = valid ? 16 * kD * 4 : 0;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(kblk), 0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vblk), 0, bytes, 0x00020000);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    r.k[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, (c * kD + 16 * j + 4 * g) * 4, 0, kNontemporal));
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      r.v[2 * t + h] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, ((4 * g + t) * kD + 64 * h + 4 * c) * 4, 0, kNontemporal));
}

// Fused append into the f32 arena (the item of the group's last chunk, before its waves
// read): a plain copy of the rows' K/V of this kv head to their slots.
template <int kThreads>
__device__ __forceinline__ void fused_append_f32(const AttnItem& it, uint32_t kh, uint32_t hkv,
                                                 uint32_t bpp_shift, const float* __restrict__ knew,
                                                 const float* __restrict__ vnew,
                                                 const uint32_t* __restrict__ kv_slot, float* kw,
                                                 float* vw) {
  const uint32_t page_size = 16u << bpp_shift;
  for (uint32_t i = threadIdx.x; i < it.nrows * 64; i += kThreads) {
    const uint32_t row = it.r0 + i / 64, ch = (i / 2) % 32;
    const bool is_k = (i & 1) == 0;
    const float* src = (is_k ? knew : vnew) + (static_cast<size_t>(row) * hkv + kh) * kD + ch * 4;
    const uint32_t slot = kv_slot[row];
    const uint32_t off = slot & (page_size - 1);
    const size_t region = (static_cast<size_t>(slot >> (bpp_shift + 4)) * hkv + kh) * page_size * kD;
    *reinterpret_cast<float4*>((is_k ? kw : vw) + region + off * kD + ch * 4) =
        *reinterpret_cast<const float4*>(src);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

__global__ __launch_bounds__(64 * kWideWaves) void paged_attn_decode_f32(
    const AttnItem* __restrict__ items, const uint32_t* pos,
    const uint32_t* __restrict__ pages, const float* kc, const float* vc,
    const float* q, float* __restrict__ out,
    float* __restrict__ part_o, float2* __restrict__ part_ml, uint32_t* __restrict__ counters,
    const float* __restrict__ knew, const float* __restrict__ vnew,
    const uint32_t* __restrict__ kv_slot, float* kw, float* vw,  // kw/vw alias kc/vc
    uint32_t part_o_bytes, uint32_t part_ml_bytes, uint32_t hq, uint32_t hkv,
    uint32_t bpp_shift, uint32_t window, float scale_log2, const SubRef* __restrict__ members) {
  __shared__ WideShared<1, false> sh;
  const AttnItem it = items[blockIdx.x];
  const uint32_t kh = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  const uint32_t G = hq / hkv;
  const uint32_t nlog = it.nrows * G;  // logical rows in the group (at most 16)

  if (knew != nullptr && it.chunk == it.nch - 1 && !(it.pref_info & kPrefixItem))
    fused_append_f32<64 * kWideWaves>(it, kh, hkv, bpp_shift, knew, vnew, kv_slot, kw, vw);

  const uint32_t nall = it.blk1 - it.blk0;
  const uint32_t wb0 = it.blk0 + nall * wave / kWideWaves;
  const uint32_t wb1 = it.blk0 + nall * (wave + 1) / kWideWaves;
  const uint32_t nblk = wb1 - wb0;
  const uint32_t bpp_mask = (1u << bpp_shift) - 1u;
  const size_t head_stride = static_cast<size_t>(16u << bpp_shift) * kD;
  const uint32_t* pt = pages + it.pt_off;
  int pid = 0;  // page id of block wb0 + lane
  if (static_cast<uint32_t>(lane) < nblk) pid = static_cast<int>(pt[(wb0 + lane) >> bpp_shift]);
  const int key_end = static_cast<int>(wb1 * 16);

  BlockRegsF32 s0, s1;
  auto load_set = [&](BlockRegsF32& r, uint32_t b) {
    const bool valid = b < nblk;
    const uint32_t page = static_cast<uint32_t>(__builtin_amdgcn_readlane(pid, static_cast<int>(valid ? b : 0)));
    const size_t o = (static_cast<size_t>(page) * hkv + kh) * head_stride +
                     static_cast<size_t>((wb0 + b) & bpp_mask) * 16 * kD;
    load_block_f32(r, kc + o, vc + o, valid, lane);
    __builtin_amdgcn_sched_barrier(0);
  };

  // This lane's column: its row position, key window and q (dims 16j + 4g + 0..3).
  const uint32_t lr = c;
  const bool has_row = lr < nlog;
  const uint32_t lrc = has_row ? lr : 0;
  const uint32_t rr = it.r0 + lrc / G, h = kh * G + lrc % G;
  const int p0 = static_cast<int>(pos[rr]);
  const int rpos = has_row ? p0 : -1;
  const int rlo = (window > 0 && p0 + 1 > static_cast<int>(window)) ? p0 + 1 - static_cast<int>(window) : 0;
  float4 qv[8];
  {
    const float* qp = q + (static_cast<size_t>(rr) * hq + h) * kD + 4 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) qv[j] = *reinterpret_cast<const float4*>(qp + 16 * j);
  }
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  load_set(s0, 0);
  load_set(s1, 1);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (!has_row) qv[j] = float4{0, 0, 0, 0};

  float m = -INFINITY, l = 0.0f;
  floatx4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = floatx4{0, 0, 0, 0};

  auto process_set = [&](const BlockRegsF32& r, uint32_t b) {
    const int kb0 = static_cast<int>((wb0 + b) * 16) + 4 * g;
    floatx4 sp[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sp[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(r.k[j].x, qv[j].x, sp[0], 0, 0, 0);
      sp[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(r.k[j].y, qv[j].y, sp[1], 0, 0, 0);
      sp[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(r.k[j].z, qv[j].z, sp[2], 0, 0, 0);
      sp[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(r.k[j].w, qv[j].w, sp[3], 0, 0, 0);
    }
    float x[4];
    float bmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kp = kb0 + i;
      const bool ok = (kp >= rlo) & (kp <= rpos) & (kp < key_end);
      x[i] = ok ? ((sp[0][i] + sp[1][i]) + (sp[2][i] + sp[3][i])) * scale_log2 : -INFINITY;
      bmax = fmaxf(bmax, x[i]);
    }
    bmax = max_xor32(max_xor16(bmax));
    const float mn = fmaxf(m, bmax);
    const bool live = mn != -INFINITY;
    float pr[4], rs = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = live ? __builtin_amdgcn_exp2f(x[i] - mn) : 0.0f;
      rs += pr[i];
    }
    rs = sum_xor32(sum_xor16(rs));
    if (__builtin_amdgcn_ballot_w64(mn != m)) {
      const float corr = live ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
      l *= corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= corr;
    }
    l += rs;
    m = mn;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) {
        const float4 vv = r.v[2 * t + mm / 4];
        const float a = (mm % 4 == 0) ? vv.x : (mm % 4 == 1) ? vv.y : (mm % 4 == 2) ? vv.z : vv.w;
        acc[mm] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, pr[t], acc[mm], 0, 0, 0);
      }
    }
  };

  for (uint32_t b = 0; b < nblk; b += 2) {
    process_set(s0, b);
    load_set(s0, b + 2);
    process_set(s1, b + 1);
    load_set(s1, b + 3);
  }

  if (g == 0) {
    sh.m[wave][c] = m;
    sh.l[wave][c] = l;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sh.o[wave][c][4 * g + i] = float4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
    sh.o[wave][c][16 + 4 * g + i] = float4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]};
  }
  __syncthreads();

  finish_item<64 * kWideWaves, 16, true>(it, kh, G, hq, hkv, nlog, out, part_o, part_ml, counters,
                                   part_o_bytes, part_ml_bytes, sh.last,
                                   [&](uint32_t lr2, uint32_t qi, float& mt, float& lt, float4& o) {
    mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWideWaves; ++w) mt = fmaxf(mt, sh.m[w][lr2]);
    lt = 0.0f;
    o = float4{0, 0, 0, 0};
    if (mt == -INFINITY) return;
#pragma unroll
    for (int w = 0; w < kWideWaves; ++w) {
      const float wt = __builtin_amdgcn_exp2f(sh.m[w][lr2] - mt);
      lt += sh.l[w][lr2] * wt;
      const float4 ow = sh.o[w][lr2][qi];
      o.x += ow.x * wt;
      o.y += ow.y * wt;
      o.z += ow.z * wt;
      o.w += ow.w * wt;
    }
  }, members);
}

}  // namespace yx
