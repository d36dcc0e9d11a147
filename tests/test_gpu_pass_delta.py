"""Device-resident pass metadata (yx_pass_begin, GPU ops/mod.rs:76-99 in the reference):
each sequence's page table keeps a device region from pass to pass, and a pass sends
only the entries that changed. Checked over decode steps (an entry per sequence that
opens a page, none otherwise), a copy-on-write step (the copied page's entry), a pass
with other groups (laid out anew, every entry sent) and a table outgrowing its region;
every pass's attention against the oracle."""

import numpy as np
import pytest

from tests.scenario import D, Scenario, close

pytestmark = pytest.mark.gpu
HQ, HKV = 8, 4


def _attend_check(hip, sc, pr, window=0):
    rows = len(pr.meta.pos)
    q = sc.draw(rows * HQ * D).reshape(rows, HQ * D)
    got = hip.attend(sc.kv, 0, q, HQ, window=window)
    want = sc.orc[0].attend(q, HQ, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"


def test_decode_steps_send_only_new_pages(hip):
    sc = Scenario(hip, pages=1024, page=16, hkv=HKV, pool_seed=5, seed=17)
    try:
        seqs = [sc.cache.new_seq() for _ in range(6)]
        sc.prefill(dict(zip(seqs, [40, 100, 15, 260, 31, 64])))
        lens = [sc.cache.seq_len(s) for s in seqs]
        for step in range(40):
            before = hip.stat("page_entries_sent")
            pr = sc.run_pass([(s, 1) for s in seqs])
            sent = hip.stat("page_entries_sent") - before
            sc.store(pr)
            # (The prefill was one pass of the same six groups in the same order, so the
            # first step already finds its regions.)
            opened = sum(1 for n in lens if n % 16 == 0)  # the new token starts a page
            assert sent == opened, f"step {step}: {sent} entries sent, {opened} pages opened"
            lens = [n + 1 for n in lens]
            _attend_check(hip, sc, pr)
        # Five groups instead of six: laid out anew, every entry of every table sent.
        before = hip.stat("page_entries_sent")
        pr = sc.run_pass([(s, 1) for s in seqs[1:]])
        sent = hip.stat("page_entries_sent") - before
        sc.store(pr)
        assert sent == sum((n + 1 + 15) // 16 for n in lens[1:])
        _attend_check(hip, sc, pr)
    finally:
        sc.kv.destroy()


def test_copy_on_write_sends_the_copied_entry(hip):
    sc = Scenario(hip, pages=256, page=16, hkv=HKV, pool_seed=6, seed=18)
    try:
        a = sc.cache.new_seq()
        sc.prefill({a: 48})  # three full pages
        cp = []
        b = sc.cache.fork(a, 48, cp)  # shares all three (whole pages: no copy)
        assert cp == []
        pr = sc.run_pass([(a, 1), (b, 1)])  # each opens a page of its own
        sc.store(pr)
        _attend_check(hip, sc, pr)
        sc.cache.truncate(b, 44)  # b's last page is again the shared third one
        b_before = list(sc.cache.seq_pages(b))
        before = hip.stat("page_entries_sent")
        copies = []
        pr = sc.run_pass([(a, 1), (b, 1)], copies)  # b writes into the shared page: a copy
        sent = hip.stat("page_entries_sent") - before
        sc.store(pr)
        assert len(copies) == 1
        b_after = list(sc.cache.seq_pages(b))
        assert b_after[:2] == b_before[:2] and b_after[2] == copies[0].dst != b_before[2]
        assert sent == 1  # the copied page's entry; a's table did not change
        _attend_check(hip, sc, pr)
    finally:
        sc.kv.destroy()


def test_tables_outgrowing_their_region_are_laid_out_again(hip):
    sc = Scenario(hip, pages=2048, page=16, hkv=HKV, pool_seed=7, seed=19)
    try:
        seqs = [sc.cache.new_seq() for _ in range(3)]
        sc.prefill(dict(zip(seqs, [16, 300, 33])))
        pr = sc.run_pass([(s, 1) for s in seqs])
        sc.store(pr)
        _attend_check(hip, sc, pr)
        # A long chunk for the first sequence (64 + more pages than its region holds),
        # then decode steps again: every pass's results against the oracle.
        for chunk in (1200, 1, 1, 900, 1):
            items = [(seqs[0], chunk)] + [(s, 1) for s in seqs[1:]]
            pr = sc.run_pass(items)
            sc.store(pr)
            _attend_check(hip, sc, pr)
            _attend_check(hip, sc, pr, window=200)
    finally:
        sc.kv.destroy()
