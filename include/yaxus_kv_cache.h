/*
 * yaxus_kv_cache.h — host-side paged KV bookkeeping behind a C ABI.
 *
 * Replaces yaxus-model's `KvCache` (crates/yaxus-model/src/kv.rs:110-353) and the
 * gather-index half of `PassMeta` (crates/yaxus-model/src/lib.rs:63-89). The page
 * size is a run-time parameter (the reference fixes `PAGE = 128`, kv.rs:17).
 *
 * Conventions: every call returns an int status (YX_OK = 0) unless stated; on error
 * `yx_cache_last_error()` gives a thread-local message. No exception crosses the ABI.
 * A null handle or a null array that the call would read or write is refused with
 * YX_ERR_INVALID; calls returning a size or an id return 0 for it and void calls do
 * nothing.
 * Operations that need pages copied append `(src, dst)` pairs to the cache's pending
 * copy list, whether or not they then succeed (kv.rs:4-7); the caller drains it with
 * `yx_cache_take_copies` and must make the copies, in order, before the next pass.
 */
#ifndef YAXUS_KV_CACHE_H
#define YAXUS_KV_CACHE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  YX_OK = 0,
  YX_ERR_INVALID = 1,     /* bad argument (empty prompt, fork beyond the end, ...) */
  YX_ERR_FULL = 2,        /* "KV cache is full" (kv.rs:283, 316, 322) */
  YX_ERR_LIMIT = 3,       /* context length exceeds max_pos (kv.rs:305) */
  YX_ERR_UNKNOWN_SEQ = 4, /* "unknown sequence" (kv.rs:278, 302) */
  YX_ERR_HIP = 5,         /* a HIP runtime call failed */
  YX_ERR_UNSUPPORTED = 6  /* a shape or dtype the kernels are not built for */
};

/* kv.rs:25, kv.rs:27 */
#define YX_MIN_REUSE 16
#define YX_MAX_CACHED 32

typedef struct yx_cache yx_cache;

/* kv.rs:35-38 `PageCopy` */
typedef struct {
  uint32_t src;
  uint32_t dst;
} yx_page_copy;

const char* yx_cache_last_error(void);

/* kv.rs:128 `KvCache::new(pages, max_pos)` (+ the page size). */
int yx_cache_create(size_t pages, size_t max_pos, size_t page_size, yx_cache** out);
void yx_cache_destroy(yx_cache* c);

/* kv.rs:140 `set_prefix_reuse` */
void yx_cache_set_prefix_reuse(yx_cache* c, int on);
/* kv.rs:154 `new_seq` */
uint64_t yx_cache_new_seq(yx_cache* c);
/* kv.rs:158 `free_seq` */
void yx_cache_free_seq(yx_cache* c, uint64_t id);
/* kv.rs:181 `clear_prefix_cache` */
void yx_cache_clear_prefix_cache(yx_cache* c);
/* kv.rs:189 `begin(prompt, copies) -> (SeqId, reused)` */
int yx_cache_begin(yx_cache* c, const uint32_t* prompt, size_t n, uint64_t* id, size_t* reused);
/* kv.rs:231 `finish` */
void yx_cache_finish(yx_cache* c, uint64_t id);
/* kv.rs:240 `seq_len` (0 for an unknown sequence) */
size_t yx_cache_seq_len(const yx_cache* c, uint64_t id);
/* kv.rs:245 `seq_tokens`: copies min(len, cap) tokens, returns len. */
size_t yx_cache_seq_tokens(const yx_cache* c, uint64_t id, uint32_t* out, size_t cap);
/* The page table of a sequence: copies min(n, cap) page ids, returns n. */
size_t yx_cache_seq_pages(const yx_cache* c, uint64_t id, uint32_t* out, size_t cap);
/* kv.rs:250, 255, 260 */
size_t yx_cache_free_pages(const yx_cache* c);
size_t yx_cache_total_pages(const yx_cache* c);
size_t yx_cache_max_pos(const yx_cache* c);
size_t yx_cache_page_size(const yx_cache* c);
/* Reference count of one page (PagePool::refs, kv.rs:49-52). */
uint32_t yx_cache_page_refs(const yx_cache* c, uint32_t page);
/* kv.rs:265 `truncate`: YX_ERR_INVALID for len > seq_len (the reference panics). */
int yx_cache_truncate(yx_cache* c, uint64_t id, size_t len);
/* kv.rs:277 `fork(id, len, copies) -> SeqId` */
int yx_cache_fork(yx_cache* c, uint64_t id, size_t len, uint64_t* out);

/*
 * kv.rs:330 `append(items, copies) -> PassRows`: item i appends counts[i] tokens
 * (taken in order from `tokens`) to sequence ids[i]. On success the pass metadata
 * is held by the cache until the next append; read it with yx_cache_pass_*.
 */
int yx_cache_append(yx_cache* c, size_t n_items, const uint64_t* ids, const size_t* counts,
                    const uint32_t* tokens);
/* PassMeta (lib.rs:63-89) of the last successful append. Each getter copies into
 * arrays the caller sized from yx_cache_pass_rows / _npages / _nitems. */
size_t yx_cache_pass_rows(const yx_cache* c);
size_t yx_cache_pass_npages(const yx_cache* c);
size_t yx_cache_pass_nitems(const yx_cache* c);
void yx_cache_pass_get(const yx_cache* c, uint32_t* ids, uint32_t* pos, uint32_t* kv_slot,
                       uint32_t* pt_off, uint32_t* pages, size_t* last);

/* Pending page copies: how many, and drain up to cap of them (returns the count taken). */
size_t yx_cache_pending_copies(const yx_cache* c);
size_t yx_cache_take_copies(yx_cache* c, yx_page_copy* out, size_t cap);

#ifdef __cplusplus
}
#endif
#endif
