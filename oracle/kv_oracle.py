"""CPU oracle (test infrastructure only) for the paged KV bookkeeping.

A pure-Python restatement of ``crates/yaxus-model/src/kv.rs`` (the whole file) with
the page size as a parameter (the reference fixes ``PAGE = 128``, kv.rs:17). It is
the checker for the shipped C++ allocator (``yaxus_amd/csrc/kv_cache.cpp``) and is
never used by it. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import anything under ``oracle/``.

Pinned by: the reference's own unit tests, restated as known-answer tests in
``tests/test_kv_host.py`` (kv.rs:365-403; lib.rs:725-775; the engine admission
tests engine/mod.rs:969-1030 at the allocator level), and by invariants checked over
random operation sequences (refcount = number of page-table occurrences, the free
list is exactly the pages with refcount 0, slots are ``pages[pos // P] * P + pos % P``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

MIN_REUSE = 16  # kv.rs:25
MAX_CACHED = 32  # kv.rs:27


class KvError(Exception):
    """An ``Err`` of the reference (``ensure!`` / ``context``)."""


@dataclass
class Seq:
    pages: list = field(default_factory=list)
    len: int = 0
    tokens: list = field(default_factory=list)


class OraclePagePool:
    """kv.rs:49-76."""

    def __init__(self, n):
        self.refs = [0] * n
        self.free = list(range(n - 1, -1, -1))

    def alloc(self):
        if not self.free:
            return None
        p = self.free.pop()
        self.refs[p] = 1
        return p

    def retain(self, p):
        self.refs[p] += 1

    def release(self, p):
        self.refs[p] -= 1
        if self.refs[p] == 0:
            self.free.append(p)

    def is_shared(self, p):
        return self.refs[p] > 1


class OraclePrefixCache:
    """kv.rs:80-107."""

    def __init__(self):
        self.entries = []  # [(id, clock)]
        self.clock = 0

    def touch(self, i):
        self.remove(i)
        self.clock += 1
        self.entries.append((i, self.clock))

    def remove(self, i):
        before = len(self.entries)
        self.entries = [e for e in self.entries if e[0] != i]
        return len(self.entries) != before

    def least_recent(self):
        if not self.entries:
            return None
        return min(self.entries, key=lambda e: e[1])[0]


class OracleKvCache:
    """kv.rs:110-353 ``KvCache``; ``copies`` lists are caller-provided like the reference."""

    def __init__(self, pages, max_pos, page):
        self.pool = OraclePagePool(pages)
        self.seqs = {}
        self.next_id = 0
        self.max_pos = max_pos
        self.P = page
        self.prefix = OraclePrefixCache()
        self.reuse = True

    def slot(self, pages, pos):  # kv.rs:20-22
        return pages[pos // self.P] * self.P + pos % self.P

    def set_prefix_reuse(self, on):  # kv.rs:140-145
        self.reuse = on
        if not on:
            self.clear_prefix_cache()

    def _insert(self, seq):  # kv.rs:147-152
        i = self.next_id
        self.next_id += 1
        self.seqs[i] = seq
        return i

    def new_seq(self):
        return self._insert(Seq())

    def free_seq(self, i):  # kv.rs:158-165
        self.prefix.remove(i)
        s = self.seqs.pop(i, None)
        if s is not None:
            for p in s.pages:
                self.pool.release(p)

    def _evict_one(self):  # kv.rs:168-172
        i = self.prefix.least_recent()
        if i is None:
            return False
        self.free_seq(i)
        return True

    def _ensure_free(self, n):  # kv.rs:176-178
        while len(self.pool.free) < n and self._evict_one():
            pass

    def clear_prefix_cache(self):
        while self._evict_one():
            pass

    def begin(self, prompt, copies):  # kv.rs:189-212
        if not prompt:
            raise KvError("empty prompt")
        bp = self._best_prefix(prompt)
        if bp is None:
            return self.new_seq(), 0
        src, keep = bp
        kept = self.prefix.remove(src)
        if keep % self.P != 0:
            self._ensure_free(1)
            if not self.pool.free:
                keep = keep // self.P * self.P
        if kept:
            self.prefix.touch(src)
        if keep >= MIN_REUSE:
            try:
                return self.fork(src, keep, copies), keep
            except KvError:
                pass
        return self.new_seq(), 0

    def _best_prefix(self, prompt):  # kv.rs:216-228
        if not self.reuse:
            return None
        best = None
        for i, _ in self.prefix.entries:
            toks = self.seqs[i].tokens
            lcp = 0
            while lcp < min(len(toks), len(prompt)) and toks[lcp] == prompt[lcp]:
                lcp += 1
            if best is None or lcp > best[1]:
                best = (i, lcp)
        if best is None:
            return None
        keep = min(best[1], len(prompt) - 1)
        return (best[0], keep) if keep >= MIN_REUSE else None

    def finish(self, i):  # kv.rs:231-238
        if not self.reuse or self.seq_len(i) < MIN_REUSE:
            self.free_seq(i)
            return
        self.prefix.touch(i)
        while len(self.prefix.entries) > MAX_CACHED and self._evict_one():
            pass

    def seq_len(self, i):
        s = self.seqs.get(i)
        return 0 if s is None else s.len

    def seq_tokens(self, i):
        s = self.seqs.get(i)
        return [] if s is None else list(s.tokens)

    def seq_pages(self, i):
        s = self.seqs.get(i)
        return [] if s is None else list(s.pages)

    def free_pages(self):
        return len(self.pool.free)

    def total_pages(self):
        return len(self.pool.refs)

    def truncate(self, i, n):  # kv.rs:265-273
        s = self.seqs.get(i)
        if s is None:
            return
        if n > s.len:
            raise KvError("truncate beyond the end")
        s.len = n
        del s.tokens[n:]
        keep = -(-n // self.P)
        for p in s.pages[keep:]:
            self.pool.release(p)
        del s.pages[keep:]

    def fork(self, i, n, copies):  # kv.rs:277-295
        src = self.seqs.get(i)
        if src is None:
            raise KvError("unknown sequence")
        if n > src.len:
            raise KvError("fork beyond the end")
        full = n // self.P
        partial = None
        if n % self.P != 0:
            partial = self.pool.alloc()
            if partial is None:
                raise KvError("KV cache is full")
        pages = list(src.pages[:full])
        for p in pages:
            self.pool.retain(p)
        if partial is not None:
            copies.append((src.pages[full], partial))
            pages.append(partial)
        return self._insert(Seq(pages, n, list(src.tokens[:n])))

    def _reserve(self, i, n, copies):  # kv.rs:299-326
        s = self.seqs.get(i)
        if s is None:
            raise KvError("unknown sequence")
        end = s.len + n
        if end > self.max_pos:
            raise KvError(f"context length {end} exceeds the limit {self.max_pos}")
        P = self.P
        need = sum(
            1
            for pi in range(s.len // P, -(-end // P))
            if pi >= len(s.pages) or self.pool.is_shared(s.pages[pi])
        )
        self._ensure_free(need)
        s = self.seqs.get(i)
        if s is None:
            raise KvError("unknown sequence")
        for pi in range(s.len // P, -(-(s.len + n) // P)):
            if pi < len(s.pages):
                p = s.pages[pi]
                if self.pool.is_shared(p):
                    q = self.pool.alloc()
                    if q is None:
                        raise KvError("KV cache is full")
                    copies.append((p, q))
                    self.pool.release(p)
                    s.pages[pi] = q
            else:
                q = self.pool.alloc()
                if q is None:
                    raise KvError("KV cache is full")
                s.pages.append(q)

    def append(self, items, copies):
        """kv.rs:330-352: returns (ids, pos, kv_slot, pt_off, pages, last)."""
        for i, toks in items:
            self._reserve(i, len(toks), copies)
        ids, pos, slot, off, pages, last = [], [], [], [], [], []
        for i, toks in items:
            s = self.seqs[i]
            o = len(pages)
            pages.extend(s.pages)
            for j, t in enumerate(toks):
                p = s.len + j
                ids.append(t)
                pos.append(p)
                slot.append(self.slot(s.pages, p))
                off.append(o)
            s.len += len(toks)
            s.tokens.extend(toks)
            if not ids:
                raise KvError("an item without tokens starts the pass")
            last.append(len(ids) - 1)
        return ids, pos, slot, off, pages, last
