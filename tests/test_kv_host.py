"""Host-side paged KV bookkeeping: the shipped allocator (C++, yaxus_amd.kv) and the
oracle (oracle/kv_oracle.py) against the reference's own unit tests, restated as
known-answer tests, and against each other over random operation sequences.

Reference tests restated here:
  kv.rs:365-383    a_shared_page_is_copied_before_it_is_written
  kv.rs:385-403    kept_sequences_are_evicted_least_recent_first
  lib.rs:741-760   reuse_falls_back_to_a_fresh_sequence_when_the_arena_is_full
  lib.rs:762-775   reuse_shares_whole_pages_without_a_free_page
  lib.rs:777-791   a_pass_beyond_max_pos_keeps_the_prefix_cache
"""

import random

import pytest

from oracle.kv_oracle import KvError as OracleError
from oracle.kv_oracle import OracleKvCache
from yaxus_amd.kv import KvCache, KvError, PageCopy

PAGE = 128  # kv.rs:17


class Product:
    """Adapter giving the product cache the oracle's (tuple-returning) interface."""

    Error = KvError

    def __init__(self, pages, max_pos, page=PAGE):
        self.c = KvCache(pages, max_pos, page)

    def __getattr__(self, name):
        return getattr(self.c, name)

    def begin(self, prompt, copies):
        cp = []
        try:
            return self.c.begin(prompt, cp)
        finally:
            copies.extend((x.src, x.dst) for x in cp)

    def fork(self, sid, n, copies):
        cp = []
        try:
            return self.c.fork(sid, n, cp)
        finally:
            copies.extend((x.src, x.dst) for x in cp)

    def append(self, items, copies):
        cp = []
        try:
            pr = self.c.append(items, cp)
        finally:
            copies.extend((x.src, x.dst) for x in cp)
        m = pr.meta
        return (list(map(int, m.ids)), list(map(int, m.pos)), list(map(int, m.kv_slot)),
                list(map(int, m.pt_off)), list(map(int, m.pages)), pr.last)


class Oracle(OracleKvCache):
    Error = OracleError

    def page_refs(self, page):
        return self.pool.refs[page]


IMPLS = [Product, Oracle]


def run(kv, sid, toks):
    copies = []
    kv.append([(sid, toks)], copies)
    return copies


@pytest.mark.parametrize("impl", IMPLS)
def test_a_shared_page_is_copied_before_it_is_written(impl):
    kv = impl(4, 1024, PAGE)
    a = kv.new_seq()
    assert run(kv, a, list(range(150))) == []
    copies = []
    # Sharing 140 tokens: page 0 shared, page 1 (partly used) copied.
    b = kv.fork(a, 140, copies)
    assert len(copies) == 1
    assert (kv.seq_len(b), kv.free_pages()) == (140, 1)
    # Writing into the shared first page of a third sequence copies it.
    c = kv.fork(a, PAGE, [])
    kv.truncate(c, 100)
    copies = run(kv, c, [7])
    assert len(copies) == 1
    assert copies[0][0] != copies[0][1]
    assert len(kv.seq_tokens(c)) == 101


@pytest.mark.parametrize("impl", IMPLS)
def test_kept_sequences_are_evicted_least_recent_first(impl):
    kv = impl(3, 1024, PAGE)
    a, b = kv.new_seq(), kv.new_seq()
    run(kv, a, [1] * 20)
    run(kv, b, [2] * 20)
    kv.finish(a)
    kv.finish(b)
    assert kv.free_pages() == 1
    # A prompt sharing `a`'s prefix reuses it and makes it the most recent.
    c, reused = kv.begin([1] * 30, [])
    assert reused == 20
    kv.free_seq(c)
    # Needing two pages evicts `b` first, then `a`.
    d = kv.new_seq()
    run(kv, d, [3] * (2 * PAGE))
    assert kv.seq_len(b) == 0
    assert kv.seq_len(a) == 20


def _prefill(kv, sid, toks, chunk=512):
    """Model::prefill's KV effect (lib.rs:475-484): chunks of at most 512 rows."""
    for i in range(0, len(toks), chunk):
        run(kv, sid, toks[i:i + chunk])


def _start(kv, prompt):
    sid, reused = kv.begin(prompt, [])
    _prefill(kv, sid, prompt[reused:])
    return sid


@pytest.mark.parametrize("impl", IMPLS)
def test_reuse_falls_back_to_a_fresh_sequence_when_the_arena_is_full(impl):
    kv = impl(2, 8192, PAGE)
    a = list(range(130))
    sid = _start(kv, a)
    kv.finish(sid)
    assert kv.free_pages() == 0
    b = a[:129] + [500, 501]
    sid, reused = kv.begin(b, [])
    # The partly used page would need a page only evicting the source gives: the
    # whole first page is shared instead, and the rest computed.
    assert reused == PAGE
    _prefill(kv, sid, b[reused:])
    assert kv.seq_len(sid) == len(b)
    assert kv.seq_tokens(sid) == b


@pytest.mark.parametrize("impl", IMPLS)
def test_reuse_shares_whole_pages_without_a_free_page(impl):
    kv = impl(2, 8192, PAGE)
    a = list(range(200))
    sid = _start(kv, a)
    kv.finish(sid)
    b = a[:PAGE] + [999]
    sid, reused = kv.begin(b, [])
    assert reused == PAGE
    _prefill(kv, sid, b[reused:])
    assert kv.seq_tokens(sid) == b


@pytest.mark.parametrize("impl", IMPLS)
def test_a_pass_beyond_max_pos_keeps_the_prefix_cache(impl):
    kv = impl(2, 200, PAGE)
    sid = _start(kv, list(range(100)))
    kv.finish(sid)
    free = kv.free_pages()
    sid, _ = kv.begin([7] * 20, [])
    with pytest.raises(impl.Error):
        _prefill(kv, sid, [7] * 300)
    assert kv.free_pages() == free


@pytest.mark.parametrize("impl", IMPLS)
def test_gather_indices_follow_the_closed_form(impl):
    """kv_slot = pages[pos // P] * P + pos % P (kv.rs:20-22), pt_off per item."""
    P = 16
    kv = impl(64, 4096, P)
    seqs = [kv.new_seq() for _ in range(3)]
    for s, n in zip(seqs, [40, 17, 1]):
        run(kv, s, [1] * n)
    ids, pos, slot, off, pages, last = kv.append([(s, [5, 6]) for s in seqs], [])
    assert last == [1, 3, 5]
    for r in range(6):
        pt = pages[off[r]:]
        assert slot[r] == pt[pos[r] // P] * P + pos[r] % P
    assert pos == [40, 41, 17, 18, 1, 2]


@pytest.mark.parametrize("impl", IMPLS)
def test_fork_then_rollback_releases_the_copied_tail(impl):
    """Speculative verify + CoW fork + rollback at the allocator level (cfg 5 shape)."""
    P = 16
    kv = impl(40, 4096, P)
    a = kv.new_seq()
    run(kv, a, list(range(37)))  # 2 full pages + 5 tokens
    copies = []
    b = kv.fork(a, 37, copies)
    assert len(copies) == 1 and copies[0][0] == kv.seq_pages(a)[2]
    assert kv.page_refs(kv.seq_pages(a)[0]) == 2
    run(kv, b, [9] * 5)  # verify 5 draft tokens
    kv.truncate(b, 37 + 2)  # keep 2 of them
    assert kv.seq_len(b) == 39 and len(kv.seq_pages(b)) == 3
    kv.truncate(b, 32)  # back to the shared whole pages: the tail copy is released
    assert len(kv.seq_pages(b)) == 2


def _state(kv, live):
    return (kv.free_pages(), [(kv.seq_len(s), kv.seq_pages(s), kv.seq_tokens(s)) for s in live])


def test_product_equals_oracle_on_random_operations():
    """The same seeded sequence of begin/append/fork/truncate/finish/free on both
    implementations: every result, copy list, error and page table is equal."""
    rnd = random.Random(20241201)
    for trial in range(40):
        P = rnd.choice([16, 32, 128])
        pages = rnd.randint(2, 40)
        max_pos = rnd.choice([P * 3, 300, 4096])
        a, b = Product(pages, max_pos, P), Oracle(pages, max_pos, P)
        live = []
        vocab = rnd.randint(2, 5)
        for step in range(120):
            op = rnd.random()
            ca, cb = [], []
            ea = eb = None
            if op < 0.25 or not live:
                prompt = [rnd.randrange(vocab) for _ in range(rnd.randint(1, 3 * P))]
                if b.seqs and rnd.random() < 0.6:
                    # Extend the tokens of a live or kept sequence: prefix reuse.
                    base = b.seqs[rnd.choice(sorted(b.seqs))].tokens
                    prompt = base[:rnd.randint(0, len(base))] + prompt[:rnd.randint(1, P)]
                try:
                    ra = a.begin(prompt, ca)
                except KvError as e:
                    ea = type(e)
                try:
                    rb = b.begin(prompt, cb)
                except OracleError as e:
                    eb = type(e)
                assert (ea is None) == (eb is None)
                if ea is None:
                    assert ra == rb
                    live.append(ra[0])
            elif op < 0.6:
                items = []
                for s in rnd.sample(live, min(len(live), rnd.randint(1, 3))):
                    items.append((s, [rnd.randrange(vocab) for _ in range(rnd.randint(1, P + 3))]))
                try:
                    ra = a.append(items, ca)
                except KvError:
                    ra = "err"
                try:
                    rb = b.append(items, cb)
                except OracleError:
                    rb = "err"
                assert ra == rb
            elif op < 0.7:
                s = rnd.choice(live)
                n = rnd.randint(0, b.seq_len(s))
                try:
                    ra = a.fork(s, n, ca)
                except KvError:
                    ra = "err"
                try:
                    rb = b.fork(s, n, cb)
                except OracleError:
                    rb = "err"
                assert ra == rb
                if ra != "err":
                    live.append(ra)
            elif op < 0.8:
                s = rnd.choice(live)
                n = rnd.randint(0, b.seq_len(s))
                a.truncate(s, n)
                b.truncate(s, n)
            elif op < 0.92:
                s = live.pop(rnd.randrange(len(live)))
                a.finish(s)
                b.finish(s)
            else:
                s = live.pop(rnd.randrange(len(live)))
                a.free_seq(s)
                b.free_seq(s)
            assert ca == cb, f"trial {trial} step {step}: copies differ"
            assert _state(a, live) == _state(b, live), f"trial {trial} step {step}"
            # Invariants: refcount = occurrences in all page tables (kept sequences
            # included); the free list is exactly the pages nobody holds.
            occ = [0] * pages
            for sq in b.seqs.values():
                for p in sq.pages:
                    occ[p] += 1
            assert occ == b.pool.refs
            assert sorted(b.pool.free) == [p for p in range(pages) if occ[p] == 0]
            assert [a.page_refs(p) for p in range(pages)] == occ


def test_random_operations_reach_prefix_reuse():
    """The differential run above does exercise reuse: count reused begins."""
    rnd = random.Random(7)
    kv = Oracle(30, 4096, 16)
    reused_total = 0
    live = []
    for _ in range(300):
        if kv.seqs and rnd.random() < 0.6:
            base = kv.seqs[rnd.choice(sorted(kv.seqs))].tokens
            prompt = base[:rnd.randint(0, len(base))] + [rnd.randrange(3)]
        else:
            prompt = [rnd.randrange(3) for _ in range(rnd.randint(1, 40))]
        try:
            s, r = kv.begin(prompt, [])
            reused_total += r > 0
            run(kv, s, prompt[r:])
            kv.finish(s)
        except OracleError:
            pass
    assert reused_total > 20


def test_product_errors_match_the_reference_messages():
    kv = KvCache(1, 100, 16)
    with pytest.raises(KvError, match="empty prompt"):
        kv.begin([], [])
    s = kv.new_seq()
    with pytest.raises(KvError, match="exceeds the limit"):
        kv.append([(s, [1] * 101)], [])
    kv.append([(s, [1] * 16)], [])
    t = kv.new_seq()
    with pytest.raises(KvError, match="KV cache is full"):
        kv.append([(t, [1])], [])
    with pytest.raises(KvError, match="fork beyond the end"):
        kv.fork(s, 17, [])
    with pytest.raises(KvError, match="unknown sequence"):
        kv.fork(12345, 1, [])
    with pytest.raises(KvError, match="truncate beyond the end"):
        kv.truncate(s, 17)
    assert PageCopy(1, 2) == PageCopy(1, 2)
