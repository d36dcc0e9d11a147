/*
 * yaxus_hip.h — the device half of yaxus's paged KV-cache path on MI355X (gfx950).
 *
 * These entry points are what a Rust FFI crate implementing yaxus's `Backend` trait
 * (crates/yaxus-model/src/lib.rs:95-171) binds for the KV path:
 *   Backend::new_kv      (lib.rs:118)  -> yx_kv_create
 *   Backend::copy_page   (lib.rs:120)  -> yx_kv_copy_pages (a batch of PageCopy, kv.rs:35)
 *   Backend::begin_pass  (lib.rs:123)  -> yx_pass_begin    (PassMeta, lib.rs:63-89)
 *   Backend::attention   (lib.rs:132)  -> yx_attention_qkv_dev (write_rows, backend-cpu
 *                                          lib.rs:359-385, then attend, lib.rs:389-427);
 *                                          or its halves: yx_qk_rope_append_dev and
 *                                          yx_attention_dev; yx_kv_append stores K/V alone
 *
 * Conventions: int status, YX_OK = 0 (codes shared with yaxus_kv_cache.h);
 * yx_last_error() returns a thread-local message; no exception crosses the ABI. Every
 * call takes a context; all device work goes, in call order, on the context's one HIP
 * stream. Calls whose pointers are host pointers are synchronous; the `_dev` variants
 * take device pointers and are asynchronous (yx_sync waits).
 *
 * The arena layout is private: per layer, K and V are `[page][kv_head][page_size][128]`
 * IEEE binary16, so one (page, kv head) is one contiguous block. head_dim is 128 (the
 * reference GPU kernels are written for 128 as well: yaxus-backend-gpu lib.rs:72).
 */
#ifndef YAXUS_HIP_H
#define YAXUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "yaxus_kv_cache.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct yx_ctx yx_ctx;
typedef struct yx_kv yx_kv;

enum { YX_DTYPE_F32 = 0, YX_DTYPE_F16 = 1 };
enum { YX_K = 0, YX_V = 1 };
/* Kernels whose launches yx_profile_read reports. */
enum { YX_KERNEL_ATTENTION = 0, YX_KERNEL_APPEND = 1, YX_KERNEL_COPY = 2, YX_KERNEL_QK_ROPE = 3 };

const char* yx_last_error(void);
int yx_device_count(int* n);

/* A context: one device, one stream, the current pass's metadata and the scratch
 * space of the attention (split-K partials and arrival counters). */
int yx_ctx_create(int device, yx_ctx** out);
int yx_ctx_destroy(yx_ctx* ctx);
int yx_sync(yx_ctx* ctx);
/* Tuning knobs: "attn_target_waves" (waves the split-K work list aims at; 0, the
 * default, means one work item per CU), "attn_max_chunk_blocks" (most 16-key blocks per
 * work item), "attn_max_tiles" (most logical rows, in units of 8 (row, q head) pairs,
 * one decode work item holds, 1-4, default 4; 3 at most with attn_decode_shape 1 unless
 * one row's q heads need 4, which then take the 16-row-tile kernel; a row's q heads
 * always fit one work item),
 * "prefill_min_rows" (rows of one sequence from which the prefill kernel is used; 0,
 * the default: automatic, the prefill kernel when a sequence has more (row, q head)
 * pairs than one decode work item holds and the pass makes at least one prefill tile
 * per 8 CUs; on the f32 arena, the kernel with the smaller time estimated from the
 * keys its decode items would read, the longest context and the pass's products),
 * "attn_decode_shape" (0, the default: automatic. Passes of more than 8 logical rows per
 * work item use the kernel with 16-row tiles and a fixed split of blocks over its waves;
 * so do one-tile passes whose work items split evenly over the waves or hold more than
 * 64 blocks; other one-tile passes use the kernel whose waves share a queue of blocks.
 * 1: the kernels with 8-row tiles and a fixed split only. 2: the 16-row-tile kernel for
 * every decode pass). "attn_cascade" (1, the default: consecutive groups of a one-tile
 * decode pass whose page tables start with the same pages, e.g. forks of one prompt,
 * attend those shared keys once for all their rows and merge that result into each
 * row's own; 0: every group reads its whole context). "attn_xcd_prefix" (1, the default:
 * the work items reading one chunk of a shared prefix are placed to run on one XCD, so
 * they share its L2; 0: in list order; results do not change). "prefill_split" (1, the default:
 * prefill tiles much longer than the average load of a workgroup slot, e.g. a chunk of
 * one long sequence, are split along keys and their partial results merged; 0: every
 * tile is one work item). "matmul_k_split" (workgroups per yx_matmul_bf16_dev output
 * tile along k, at most 64; 0, the default: automatic; it changes the result only by
 * the order of the f32 additions), "argmax_slices" (workgroups per yx_argmax_rows_dev
 * row, at most 1024; 0, the default: automatic; the result does not change) and
 * "prefill_f32_waves" (the f32 arena's prefill tiles: 8 waves of 16 logical rows or 4;
 * 0, the default: 4 when every sequence of the pass has at most 64 logical rows). Setting an
 * option drops cached work lists. Values are positive; 0 is accepted for
 * attn_target_waves, attn_decode_shape, attn_cascade, attn_xcd_prefix, prefill_split, prefill_min_rows,
 * matmul_k_split, argmax_slices and prefill_f32_waves (which takes 0, 4 or 8). */
int yx_ctx_set_option(yx_ctx* ctx, const char* key, long value);
/* Counters of the context since its creation: "page_entries_sent" (page-table entries
 * yx_pass_begin uploaded), "page_runs_sent" (runs of consecutive entries they formed)
 * "prefill_split_tiles" (prefill tiles split along keys in the work lists built) and
 * "prefill_plans" (work lists built as prefill tiles rather than decode items).
 * A pass whose groups keep their order and fit the device regions of the previous pass
 * sends only the entries that changed. */
int yx_ctx_get_stat(yx_ctx* ctx, const char* key, uint64_t* out);

/* Backend::new_kv (lib.rs:118; GPU ops/mod.rs:42-66): `layers` layers of `pages`
 * pages of `page_size` tokens (a multiple of 16), zeroed. dtype YX_DTYPE_F16 (binary16,
 * the fast path) or YX_DTYPE_F32 (the reference's own K/V precision: stores are exact,
 * attention runs on f32 MFMAs: split-K decode items of at most 16 (row, q head) pairs,
 * or prefill tiles of 128 or 64, chosen as the options prefill_min_rows and
 * prefill_f32_waves of yx_ctx_set_option describe;
 * at most 16 q heads per KV head; write_rows as its own launch). */
int yx_kv_create(yx_ctx* ctx, size_t layers, size_t pages, size_t page_size, size_t hkv,
                 size_t head_dim, int dtype, yx_kv** out);
int yx_kv_destroy(yx_ctx* ctx, yx_kv* kv);
/* Device pointer of one layer's K or V arena (for fills and device-side tools). */
int yx_kv_layer_ptr(yx_kv* kv, size_t layer, int which, void** out);
size_t yx_kv_page_bytes(const yx_kv* kv);

/* Backend::copy_page (lib.rs:120; CPU lib.rs:472-479), batched: page src[i] -> dst[i]
 * in every layer, K and V, in list order (a later copy sees an earlier one's result). */
int yx_kv_copy_pages(yx_ctx* ctx, yx_kv* kv, const uint32_t* src, const uint32_t* dst, size_t n);

/* Raw page contents, `[n][hkv][page_size][128]` binary16 bits (f32 bits for an f32
 * arena), synchronous. */
int yx_kv_read_pages(yx_ctx* ctx, yx_kv* kv, size_t layer, const uint32_t* pages, size_t n,
                     void* k_out, void* v_out);
int yx_kv_write_pages(yx_ctx* ctx, yx_kv* kv, size_t layer, const uint32_t* pages, size_t n,
                      const void* k_in, const void* v_in);

/* Backend::begin_pass (lib.rs:123; GPU ops/mod.rs:76-99): the rows of the next pass.
 * Rows of one sequence are consecutive, share pt_off and have consecutive positions.
 * The positions, slots and the page-table entries that differ from what the device
 * holds (the device keeps each sequence's table in a region of its own from pass to
 * pass), together with the work lists of the attention calls the previous pass made,
 * go to the device as one copy on the context's stream. */
int yx_pass_begin(yx_ctx* ctx, size_t rows, const uint32_t* pos, const uint32_t* kv_slot,
                  const uint32_t* pt_off, const uint32_t* pages, size_t npages);

/* The K/V store of write_rows (backend-cpu lib.rs:378-383; QK_ROPE's store,
 * yaxus-backend-gpu shaders.rs:285-341): k and v are `[rows][hkv][128]` f32, rounded
 * to binary16 (nearest-even) and scattered to each row's kv_slot of `layer`. */
int yx_kv_append(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* k, const float* v);
int yx_kv_append_dev(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* k, const float* v);

/* write_rows (backend-cpu lib.rs:359-385; QK_ROPE, yaxus-backend-gpu shaders.rs:285-341),
 * device pointers: per row of the pass, qkv `[rows][(hq + 2 hkv) * 128]` f32 holds the
 * q heads, then the k heads, then the v heads. Each q and k head is RMS-normalised
 * (weights q_norm / k_norm `[128]`, offset 1, eps) and rotated by half-split RoPE at the
 * row's position; q goes to q_out `[rows][hq * 128]` f32, k and the raw v to the row's
 * kv_slot of `layer` (binary16, nearest even). rope_cs is the layer's table
 * `[rope_len][64]` cos then `[rope_len][64]` sin, as Rope::cos_sin (config.rs:213-219)
 * fills it and the reference GPU backend uploads it (ops/attention.rs:112-120); every
 * row's position must be below rope_len. The results carry the CPU backend's bits. */
int yx_qk_rope_append_dev(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* qkv,
                          const float* q_norm, const float* k_norm, const float* rope_cs,
                          size_t rope_len, float eps, size_t hq, size_t hkv, float* q_out);

/* Backend::attention in full (lib.rs:132; backend-cpu lib.rs:516-530: write_rows then
 * attend), device pointers, arguments as yx_qk_rope_append_dev and yx_attention_dev.
 * A one-tile decode pass (each group's rows in one work item chain) takes one launch:
 * the attention kernel normalises and rotates its rows' q heads into LDS and the
 * group's last work item stores the rows' K/V. A prefill pass takes two: write_rows for
 * the key and value heads, then the prefill kernel, which normalises and rotates its q
 * heads itself. Other passes run write_rows, then attention. Every path has write_rows'
 * bits. out `[rows][hq * 128]` f32. */
int yx_attention_qkv_dev(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* qkv,
                         const float* q_norm, const float* k_norm, const float* rope_cs,
                         size_t rope_len, float eps, float* out, size_t hq, size_t hkv,
                         size_t window, float scale);

/* attend (backend-cpu lib.rs:389-427; ATTN_SPLIT + ATTN_COMBINE, shaders.rs:1466-1637):
 * causal GQA attention of q `[rows][hq][128]` f32 over each row's keys `[lo, pos]`,
 * lo = pos + 1 - window when window > 0 and pos + 1 > window, else 0. out is
 * `[rows][hq][128]` f32. `scale` multiplies q.k (the reference uses 1/sqrt(128)). */
int yx_attention(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* q, float* out, size_t hq,
                 size_t hkv, size_t window, float scale);
int yx_attention_dev(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* q, float* out,
                     size_t hq, size_t hkv, size_t window, float scale);

/* Backend::attention's KV half in one launch (lib.rs:132; backend-cpu lib.rs:516-530):
 * stores the rows' k, v (`[rows][hkv][128]` f32, as yx_kv_append) and then attends
 * as yx_attention, the rows seeing their own and earlier rows' new keys. */
int yx_attention_append(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* k, const float* v,
                        const float* q, float* out, size_t hq, size_t hkv, size_t window,
                        float scale);
int yx_attention_append_dev(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* k,
                            const float* v, const float* q, float* out, size_t hq, size_t hkv,
                            size_t window, float scale);

/* No counterpart in the reference: yx_attention_append_dev for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same kernels, arguments and results; the split-K partials and arrival
 * counters live in the library's static device scratch (16 MiB per GPU: 1 MiB of
 * counters, 8192 of them, one per 128-byte line; a 2 MiB region for work lists; the
 * rest for partials; held until the process ends) instead of buffers of the context,
 * so the call makes no device or pinned-host allocation. The work list is the one
 * yx_pass_begin put on the device when the previous pass made the same call (a decode
 * loop's steady state), else it is sent once per pass into the scratch's list region
 * from the pass's pinned staging. A pass whose work lists or partials do not fit is
 * refused with YX_ERR_UNSUPPORTED. Every call on a GPU shares that GPU's scratch: when a
 * call comes from another context than the last one, its stream first waits for the
 * other context's stream (an event, no allocation), so contexts take turns; under graph
 * capture such a hand-over cannot be recorded and is refused (make one eager call
 * first). Calls that overlap in any other way race. */
int yx_attention_append_noalloc(yx_ctx* ctx, yx_kv* kv, size_t layer, const float* k,
                                const float* v, const float* q, float* out, size_t hq,
                                size_t hkv, size_t window, float scale);

/* The step after the attention (device pointers, asynchronous). Backend::matmul with a
 * bf16 weight (lib.rs:133; backend-cpu lib.rs:234-248, 314-345), e.g. the output
 * projection o_proj: out `[t][n]` f32 = x `[t][k]` f32 times w `[n][k]` (bf16 bits)
 * transposed; k a multiple of 8, x and w 16-byte aligned. Every product is exact (x in
 * three bf16 parts), the sums are f32. */
int yx_matmul_bf16_dev(yx_ctx* ctx, const float* x, const uint16_t* w, float* out, size_t t,
                       size_t k, size_t n);
/* SyncReadback::argmax_rows (lib.rs:182; backend-cpu lib.rs:432-440, 556-558): out[r] =
 * the first index of the largest value of row r of logits `[rows][cols]` f32; NaN is
 * never chosen, and a row with nothing above -inf gives 0. out is a device array of
 * `rows` u32. */
int yx_argmax_rows_dev(yx_ctx* ctx, const float* logits, size_t rows, size_t cols, uint32_t* out);

/* Device memory and copies on the context's stream (h2d/d2h are synchronous). */
int yx_dev_alloc(yx_ctx* ctx, size_t bytes, void** out);
int yx_dev_free(yx_ctx* ctx, void* p);
/* Pinned (page-locked) host memory, for callers whose data crosses PCIe every layer (a
 * wrapped host backend's qkv and attention output): copies from and to it run at DMA
 * speed, where pageable memory is staged through a driver buffer first. */
int yx_host_alloc(yx_ctx* ctx, size_t bytes, void** out);
int yx_host_free(yx_ctx* ctx, void* p);
int yx_memcpy_h2d(yx_ctx* ctx, void* dst, const void* src, size_t bytes);
int yx_memcpy_d2h(yx_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Plain device copy kernel (also the reference point for HBM byte counters). */
int yx_dev_copy(yx_ctx* ctx, void* dst, const void* src, size_t bytes);
/* XOR of every 8-byte word of a device buffer (size and pointer 16-byte aligned),
 * synchronous: an order-independent checksum of device data, and a read-only pass over
 * the buffer (the read-side reference point for the HBM byte counters). */
int yx_dev_checksum(yx_ctx* ctx, const void* src, size_t bytes, uint64_t* out);
/* Synthetic N(0,1) values: splitmix64 -> Box-Muller, element i of stream `seed` at
 * index offset + i (see yaxus_amd/data.py for the definition); dtype f32 or f16. */
int yx_fill_normal(yx_ctx* ctx, void* dst, size_t n, int dtype, uint64_t seed, uint64_t offset);

/* HIP graph of the calls made between begin and end on the context's stream (each
 * must have run once before, so its work list is on the device); launch replays it.
 * The kernels leave their arrival counters at zero, so replays need no memset. A new
 * pass, an option, a destroyed arena or a grown scratch buffer since the capture makes
 * launch fail with YX_ERR_INVALID (the graph would read memory that moved): capture
 * again. Arenas and caller buffers the graph reads must stay allocated. */
int yx_graph_begin(yx_ctx* ctx);
int yx_graph_end(yx_ctx* ctx);
int yx_graph_launch(yx_ctx* ctx);

/* Timing with HIP events on the context's stream. */
int yx_timer_start(yx_ctx* ctx);
int yx_timer_stop(yx_ctx* ctx, float* ms);
/* When on, every launch of the kernels above is bracketed by an event pair;
 * yx_profile_read waits, returns the summed duration and launch count of one kernel
 * since the last read, and resets them. */
int yx_profile_enable(yx_ctx* ctx, int on);
int yx_profile_read(yx_ctx* ctx, int kernel, double* total_ms, uint64_t* launches);

#ifdef __cplusplus
}
#endif
#endif
