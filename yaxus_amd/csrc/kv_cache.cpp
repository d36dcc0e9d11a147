// Host-side paged KV bookkeeping: the page pool with reference counts, the kept
// (finished) sequences for prefix reuse, fork / copy-on-write and the construction of
// a pass's gather indices.
//
// Semantics follow crates/yaxus-model/src/kv.rs (whole file); each method cites the
// function it restates. The page size is a parameter instead of the constant
// `PAGE = 128` (kv.rs:17). Page ids, refcounts, eviction order and copies must equal
// the reference's exactly: they are compared bit for bit with an independent
// restatement in the tests.
#include "../../include/yaxus_kv_cache.h"

#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

struct Seq {
  std::vector<uint32_t> pages;
  size_t len = 0;
  std::vector<uint32_t> tokens;  // tokens.size() == len
};

// kv.rs:49-76. Free list is a LIFO stack seeded n-1 .. 0, so pages come out 0, 1, 2, ...
struct PagePool {
  std::vector<uint32_t> refs;
  std::vector<uint32_t> free_list;

  explicit PagePool(size_t n) : refs(n, 0) {
    free_list.reserve(n);
    for (size_t i = n; i-- > 0;) free_list.push_back(static_cast<uint32_t>(i));
  }
  bool alloc(uint32_t* p) {
    if (free_list.empty()) return false;
    *p = free_list.back();
    free_list.pop_back();
    refs[*p] = 1;
    return true;
  }
  void retain(uint32_t p) { refs[p] += 1; }
  void release(uint32_t p) {
    if (--refs[p] == 0) free_list.push_back(p);
  }
  bool is_shared(uint32_t p) const { return refs[p] > 1; }
};

// kv.rs:80-107: kept sequences by last use (a vector scanned linearly, insertion order
// kept: `best_prefix` takes the first of equal prefixes in this order).
struct PrefixCache {
  std::vector<std::pair<uint64_t, uint64_t>> entries;  // (seq, clock)
  uint64_t clock = 0;

  void touch(uint64_t id) {
    remove(id);
    clock += 1;
    entries.emplace_back(id, clock);
  }
  bool remove(uint64_t id) {
    size_t before = entries.size();
    size_t w = 0;
    for (size_t r = 0; r < entries.size(); ++r)
      if (entries[r].first != id) entries[w++] = entries[r];
    entries.resize(w);
    return w != before;
  }
  bool least_recent(uint64_t* id) const {
    if (entries.empty()) return false;
    size_t best = 0;
    for (size_t i = 1; i < entries.size(); ++i)
      if (entries[i].second < entries[best].second) best = i;
    *id = entries[best].first;
    return true;
  }
};

size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

}  // namespace

struct yx_cache {
  PagePool pool;
  std::unordered_map<uint64_t, Seq> seqs;
  uint64_t next_id = 0;
  size_t max_pos;
  size_t page;
  PrefixCache prefix;
  bool reuse = true;
  std::vector<yx_page_copy> copies;
  // PassMeta of the last append (lib.rs:63-89) and the last row of each item.
  std::vector<uint32_t> ids, pos, kv_slot, pt_off, pass_pages;
  std::vector<size_t> last;

  yx_cache(size_t pages, size_t max_pos_, size_t page_)
      : pool(pages), max_pos(max_pos_), page(page_) {}

  // kv.rs:20-22
  uint32_t slot(const std::vector<uint32_t>& pages, size_t p) const {
    return static_cast<uint32_t>(pages[p / page] * page + p % page);
  }

  uint64_t insert(Seq s) {
    uint64_t id = next_id++;
    seqs.emplace(id, std::move(s));
    return id;
  }

  // kv.rs:158-165
  void free_seq(uint64_t id) {
    prefix.remove(id);
    auto it = seqs.find(id);
    if (it == seqs.end()) return;
    for (uint32_t p : it->second.pages) pool.release(p);
    seqs.erase(it);
  }

  // kv.rs:168-172
  bool evict_one() {
    uint64_t id;
    if (!prefix.least_recent(&id)) return false;
    free_seq(id);
    return true;
  }

  // kv.rs:176-178
  void ensure_free(size_t n) {
    while (pool.free_list.size() < n && evict_one()) {
    }
  }

  void clear_prefix_cache() {
    while (evict_one()) {
    }
  }

  // kv.rs:216-228
  bool best_prefix(const uint32_t* prompt, size_t n, uint64_t* id, size_t* keep) const {
    if (!reuse) return false;
    bool have = false;
    uint64_t best_id = 0;
    size_t best_lcp = 0;
    for (const auto& e : prefix.entries) {
      const Seq& s = seqs.at(e.first);
      size_t lcp = 0;
      size_t lim = s.tokens.size() < n ? s.tokens.size() : n;
      while (lcp < lim && s.tokens[lcp] == prompt[lcp]) ++lcp;
      if (!have || lcp > best_lcp) {
        have = true;
        best_id = e.first;
        best_lcp = lcp;
      }
    }
    if (!have) return false;
    size_t k = best_lcp < n - 1 ? best_lcp : n - 1;
    if (k < YX_MIN_REUSE) return false;
    *id = best_id;
    *keep = k;
    return true;
  }

  // kv.rs:277-295
  int fork(uint64_t id, size_t len, uint64_t* out) {
    auto it = seqs.find(id);
    if (it == seqs.end()) return fail(YX_ERR_UNKNOWN_SEQ, "unknown sequence");
    if (len > it->second.len) return fail(YX_ERR_INVALID, "fork beyond the end");
    size_t full = len / page;
    bool partial = len % page != 0;
    uint32_t dst = 0;
    if (partial && !pool.alloc(&dst)) return fail(YX_ERR_FULL, "KV cache is full");
    const Seq& src = it->second;
    Seq s;
    s.pages.assign(src.pages.begin(), src.pages.begin() + full);
    for (uint32_t p : s.pages) pool.retain(p);
    if (partial) {
      copies.push_back({src.pages[full], dst});
      s.pages.push_back(dst);
    }
    s.tokens.assign(src.tokens.begin(), src.tokens.begin() + len);
    s.len = len;
    *out = insert(std::move(s));
    return YX_OK;
  }

  // kv.rs:189-212
  int begin(const uint32_t* prompt, size_t n, uint64_t* id, size_t* reused) {
    if (n == 0) return fail(YX_ERR_INVALID, "empty prompt");
    uint64_t src;
    size_t keep;
    if (!best_prefix(prompt, n, &src, &keep)) {
      *id = insert(Seq{});
      *reused = 0;
      return YX_OK;
    }
    // Whole pages are shared; a partly used last page needs a free page. Room is made
    // without evicting `src` (taken out of the kept list meanwhile); without a page,
    // only the whole pages are reused.
    bool kept = prefix.remove(src);
    if (keep % page != 0) {
      ensure_free(1);
      if (pool.free_list.empty()) keep = keep / page * page;
    }
    if (kept) prefix.touch(src);
    if (keep >= YX_MIN_REUSE) {
      uint64_t s;
      if (fork(src, keep, &s) == YX_OK) {
        *id = s;
        *reused = keep;
        return YX_OK;
      }
    }
    *id = insert(Seq{});
    *reused = 0;
    return YX_OK;
  }

  // kv.rs:231-238
  void finish(uint64_t id) {
    auto it = seqs.find(id);
    size_t len = it == seqs.end() ? 0 : it->second.len;
    if (!reuse || len < YX_MIN_REUSE) {
      free_seq(id);
      return;
    }
    prefix.touch(id);
    while (prefix.entries.size() > YX_MAX_CACHED && evict_one()) {
    }
  }

  // kv.rs:265-273
  int truncate(uint64_t id, size_t len) {
    auto it = seqs.find(id);
    if (it == seqs.end()) return YX_OK;
    Seq& s = it->second;
    if (len > s.len) return fail(YX_ERR_INVALID, "truncate beyond the end");
    s.len = len;
    s.tokens.resize(len);
    size_t keep = div_ceil(len, page);
    for (size_t i = keep; i < s.pages.size(); ++i) pool.release(s.pages[i]);
    if (s.pages.size() > keep) s.pages.resize(keep);
    return YX_OK;
  }

  // kv.rs:299-326
  int reserve(uint64_t id, size_t n) {
    auto it = seqs.find(id);
    if (it == seqs.end()) return fail(YX_ERR_UNKNOWN_SEQ, "unknown sequence");
    size_t need = 0;
    {
      const Seq& s = it->second;
      size_t end = s.len + n;
      // Checked before evicting anything: a pass that cannot run keeps the cache.
      if (end > max_pos) {
        char buf[128];
        snprintf(buf, sizeof buf, "context length %zu exceeds the limit %zu", end, max_pos);
        return fail(YX_ERR_LIMIT, buf);
      }
      for (size_t pi = s.len / page; pi < div_ceil(end, page); ++pi)
        if (pi >= s.pages.size() || pool.is_shared(s.pages[pi])) ++need;
    }
    ensure_free(need);
    it = seqs.find(id);
    if (it == seqs.end()) return fail(YX_ERR_UNKNOWN_SEQ, "unknown sequence");
    Seq& s = it->second;
    for (size_t pi = s.len / page; pi < div_ceil(s.len + n, page); ++pi) {
      if (pi < s.pages.size()) {
        uint32_t p = s.pages[pi];
        if (pool.is_shared(p)) {
          uint32_t q;
          if (!pool.alloc(&q)) return fail(YX_ERR_FULL, "KV cache is full");
          copies.push_back({p, q});
          pool.release(p);
          s.pages[pi] = q;
        }
      } else {
        uint32_t q;
        if (!pool.alloc(&q)) return fail(YX_ERR_FULL, "KV cache is full");
        s.pages.push_back(q);
      }
    }
    return YX_OK;
  }

  // kv.rs:330-352
  int append(size_t n_items, const uint64_t* item_ids, const size_t* counts,
             const uint32_t* tokens) {
    for (size_t i = 0; i < n_items; ++i) {
      int rc = reserve(item_ids[i], counts[i]);
      if (rc != YX_OK) return rc;
    }
    std::vector<uint32_t> m_ids, m_pos, m_slot, m_off, m_pages;
    std::vector<size_t> m_last;
    const uint32_t* t = tokens;
    for (size_t i = 0; i < n_items; ++i) {
      Seq& s = seqs.at(item_ids[i]);
      uint32_t off = static_cast<uint32_t>(m_pages.size());
      m_pages.insert(m_pages.end(), s.pages.begin(), s.pages.end());
      for (size_t j = 0; j < counts[i]; ++j) {
        size_t p = s.len + j;
        m_ids.push_back(t[j]);
        m_pos.push_back(static_cast<uint32_t>(p));
        m_slot.push_back(slot(s.pages, p));
        m_off.push_back(off);
      }
      s.len += counts[i];
      s.tokens.insert(s.tokens.end(), t, t + counts[i]);
      t += counts[i];
      if (m_ids.empty()) return fail(YX_ERR_INVALID, "an item without tokens starts the pass");
      m_last.push_back(m_ids.size() - 1);
    }
    ids.swap(m_ids);
    pos.swap(m_pos);
    kv_slot.swap(m_slot);
    pt_off.swap(m_off);
    pass_pages.swap(m_pages);
    last.swap(m_last);
    return YX_OK;
  }
};

extern "C" {

const char* yx_cache_last_error(void) { return g_err.c_str(); }

int yx_cache_create(size_t pages, size_t max_pos, size_t page_size, yx_cache** out) {
  if (!out) return fail(YX_ERR_INVALID, "null output");
  if (page_size == 0) return fail(YX_ERR_INVALID, "page size must be positive");
  if (pages > 0xffffffffull) return fail(YX_ERR_INVALID, "page ids are 32-bit");
  if (pages > 0xffffffffull / page_size) return fail(YX_ERR_INVALID, "arena slots are 32-bit");
  try {
    *out = new yx_cache(pages, max_pos, page_size);
  } catch (...) {
    return fail(YX_ERR_INVALID, "allocation failed");
  }
  return YX_OK;
}

void yx_cache_destroy(yx_cache* c) { delete c; }

void yx_cache_set_prefix_reuse(yx_cache* c, int on) {
  if (!c) return;
  c->reuse = on != 0;
  if (!c->reuse) c->clear_prefix_cache();
}

uint64_t yx_cache_new_seq(yx_cache* c) { return c ? c->insert(Seq{}) : 0; }
void yx_cache_free_seq(yx_cache* c, uint64_t id) {
  if (c) c->free_seq(id);
}
void yx_cache_clear_prefix_cache(yx_cache* c) {
  if (c) c->clear_prefix_cache();
}

int yx_cache_begin(yx_cache* c, const uint32_t* prompt, size_t n, uint64_t* id, size_t* reused) {
  if (!c || !id || !reused || (n && !prompt)) return fail(YX_ERR_INVALID, "null argument");
  try {
    return c->begin(prompt, n, id, reused);
  } catch (...) {
    return fail(YX_ERR_INVALID, "internal error in begin");
  }
}

void yx_cache_finish(yx_cache* c, uint64_t id) {
  if (c) c->finish(id);
}

size_t yx_cache_seq_len(const yx_cache* c, uint64_t id) {
  if (!c) return 0;
  auto it = c->seqs.find(id);
  return it == c->seqs.end() ? 0 : it->second.len;
}

size_t yx_cache_seq_tokens(const yx_cache* c, uint64_t id, uint32_t* out, size_t cap) {
  if (!c) return 0;
  if (!out) cap = 0;
  auto it = c->seqs.find(id);
  if (it == c->seqs.end()) return 0;
  const auto& t = it->second.tokens;
  size_t n = t.size() < cap ? t.size() : cap;
  if (n) memcpy(out, t.data(), n * sizeof(uint32_t));
  return t.size();
}

size_t yx_cache_seq_pages(const yx_cache* c, uint64_t id, uint32_t* out, size_t cap) {
  if (!c) return 0;
  if (!out) cap = 0;
  auto it = c->seqs.find(id);
  if (it == c->seqs.end()) return 0;
  const auto& p = it->second.pages;
  size_t n = p.size() < cap ? p.size() : cap;
  if (n) memcpy(out, p.data(), n * sizeof(uint32_t));
  return p.size();
}

size_t yx_cache_free_pages(const yx_cache* c) { return c ? c->pool.free_list.size() : 0; }
size_t yx_cache_total_pages(const yx_cache* c) { return c ? c->pool.refs.size() : 0; }
size_t yx_cache_max_pos(const yx_cache* c) { return c ? c->max_pos : 0; }
size_t yx_cache_page_size(const yx_cache* c) { return c ? c->page : 0; }
uint32_t yx_cache_page_refs(const yx_cache* c, uint32_t page) {
  return c && page < c->pool.refs.size() ? c->pool.refs[page] : 0;
}

int yx_cache_truncate(yx_cache* c, uint64_t id, size_t len) {
  if (!c) return fail(YX_ERR_INVALID, "null cache");
  return c->truncate(id, len);
}

int yx_cache_fork(yx_cache* c, uint64_t id, size_t len, uint64_t* out) {
  if (!c || !out) return fail(YX_ERR_INVALID, "null argument");
  try {
    return c->fork(id, len, out);
  } catch (...) {
    return fail(YX_ERR_INVALID, "internal error in fork");
  }
}

int yx_cache_append(yx_cache* c, size_t n_items, const uint64_t* ids, const size_t* counts,
                    const uint32_t* tokens) {
  if (!c || (n_items && (!ids || !counts))) return fail(YX_ERR_INVALID, "null argument");
  size_t total = 0;
  for (size_t i = 0; i < n_items; ++i) total += counts[i];
  if (total && !tokens) return fail(YX_ERR_INVALID, "null tokens");
  try {
    return c->append(n_items, ids, counts, tokens);
  } catch (...) {
    return fail(YX_ERR_INVALID, "internal error in append");
  }
}

size_t yx_cache_pass_rows(const yx_cache* c) { return c ? c->ids.size() : 0; }
size_t yx_cache_pass_npages(const yx_cache* c) { return c ? c->pass_pages.size() : 0; }
size_t yx_cache_pass_nitems(const yx_cache* c) { return c ? c->last.size() : 0; }

void yx_cache_pass_get(const yx_cache* c, uint32_t* ids, uint32_t* pos, uint32_t* kv_slot,
                       uint32_t* pt_off, uint32_t* pages, size_t* last) {
  if (!c) return;
  size_t r = c->ids.size();
  if (ids && r) memcpy(ids, c->ids.data(), r * 4);
  if (pos && r) memcpy(pos, c->pos.data(), r * 4);
  if (kv_slot && r) memcpy(kv_slot, c->kv_slot.data(), r * 4);
  if (pt_off && r) memcpy(pt_off, c->pt_off.data(), r * 4);
  if (pages && !c->pass_pages.empty())
    memcpy(pages, c->pass_pages.data(), c->pass_pages.size() * 4);
  if (last && !c->last.empty()) memcpy(last, c->last.data(), c->last.size() * sizeof(size_t));
}

size_t yx_cache_pending_copies(const yx_cache* c) { return c ? c->copies.size() : 0; }

size_t yx_cache_take_copies(yx_cache* c, yx_page_copy* out, size_t cap) {
  if (!c) return 0;
  if (!out) cap = 0;
  size_t n = c->copies.size() < cap ? c->copies.size() : cap;
  if (n) memcpy(out, c->copies.data(), n * sizeof(yx_page_copy));
  c->copies.erase(c->copies.begin(), c->copies.begin() + n);
  return n;
}

}  // extern "C"
