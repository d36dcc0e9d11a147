"""Whole steps of the benchmark configurations at full size, against the oracle.

Where tests/test_gpu_fullsize.py checks one layer of each configuration, these run a
configuration's step over all of its layers (distinct arenas, as the benchmark does) and
check every layer, and carry configuration 5 on past its verify pass: the copy-on-write
forks of the partly filled tail page, the seeded rollback and the decode step after it
(crates/yaxus-model/src/kv.rs:265-326).

Page tables, copy lists, rollback lengths and pass metadata are compared bit for bit
with the allocator oracle (oracle/kv_oracle.py) run through the same operations; the
copied pages' bytes are compared with their sources' on the device in every layer; the
appended K/V with their binary16 roundings; attention within 2e-3 abs + 1e-3 rel of the
attention oracle over the same K/V bits.
"""

import os

import numpy as np
import pytest

import bench
from oracle.attn import OracleArena, f32_to_f16_bits, normal
from oracle.kv_oracle import OracleKvCache
from tests.scenario import close
from yaxus_amd import KvCache
from yaxus_amd.data import permutation, uniform_ints

pytestmark = pytest.mark.gpu
D, HQ, HKV, PAGE = bench.D, bench.HQ, bench.HKV, bench.PAGE
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _mirror(orc, kv, layer, pages):
    """Copies the device pages of `layer` into the oracle arena (slot-major)."""
    pages = np.unique(np.asarray(pages, np.uint32))
    for part in np.array_split(pages, max(1, len(pages) // 2048)):
        k, v = kv.read_pages(layer, part)
        slots = (part.astype(np.int64)[:, None] * PAGE + np.arange(PAGE)).reshape(-1)
        orc.k[slots] = k.transpose(0, 2, 1, 3).reshape(len(part) * PAGE, HKV * D)
        orc.v[slots] = v.transpose(0, 2, 1, 3).reshape(len(part) * PAGE, HKV * D)


def _check_appended(kv, layer, meta, k, v):
    slots = np.asarray(meta.kv_slot, np.int64)
    pages = np.unique(slots // PAGE).astype(np.uint32)
    kk, vv = kv.read_pages(layer, pages)
    index = {int(p): i for i, p in enumerate(pages)}
    for r, s in enumerate(slots):
        i, off = index[int(s // PAGE)], int(s % PAGE)
        assert np.array_equal(kk[i, :, off, :], f32_to_f16_bits(k[r])), f"layer {layer}: K of row {r}"
        assert np.array_equal(vv[i, :, off, :], f32_to_f16_bits(v[r])), f"layer {layer}: V of row {r}"


def _step(hip, kv, meta, windows, seed):
    """One decode/verify step: the fused append + attention of every layer (device
    inputs, as one step of a model), then every layer checked against the oracle."""
    rows = len(meta.pos)
    layers = len(windows)
    ins = []
    for l in range(layers):
        k = normal(rows * HKV * D, seed, (3 * l) * rows * HQ * D).reshape(rows, HKV, D)
        v = normal(rows * HKV * D, seed, (3 * l + 1) * rows * HQ * D).reshape(rows, HKV, D)
        q = normal(rows * HQ * D, seed, (3 * l + 2) * rows * HQ * D).reshape(rows, HQ * D)
        ins.append((hip.tensor(k.shape).upload(k), hip.tensor(v.shape).upload(v),
                    hip.tensor(q.shape).upload(q), hip.tensor((rows, HQ * D)), k, v, q))
    hip.begin_pass(meta)
    for l in range(layers):
        dk, dv, dq, do, *_ = ins[l]
        hip.attend_append(kv, l, dk, dv, dq, HQ, window=windows[l], out=do)
    hip.sync()
    orc = None
    try:
        for l in range(layers):
            dk, dv, dq, do, k, v, q = ins[l]
            got = do.numpy()
            _check_appended(kv, l, meta, k, v)
            if orc is None:
                orc = OracleArena(kv.pages, PAGE, HKV, D, f16=True)
            _mirror(orc, kv, l, meta.pages)
            want = orc.attend(q, HQ, meta.pos, meta.pt_off, meta.pages, window=windows[l],
                              threads=THREADS)
            ok = close(got, want)
            assert ok.all(), (f"layer {l} (window {windows[l]}): max abs err "
                              f"{np.abs(got - want).max()}")
    finally:
        for t in ins:
            for d in t[:4]:
                d.free()


def test_cfg2_all_24_layers(hip):
    """cfg2's decode step over its 24 layers (one shared 1024-token prefix, suffixes
    U[512, 3072]), every layer against the oracle."""
    _, pr, pool, _ = bench.cfg2_pass(KvCache)
    kv = hip.new_kv(24, pool, PAGE, HKV, D)
    try:
        bench._fill_arena(hip, kv, 24, bench.SEED + 21)
        _step(hip, kv, pr.meta, [0] * 24, bench.SEED + 22)
    finally:
        kv.destroy()


def test_cfg4_32_layer_interleaved_step(hip):
    """cfg4's whole decode step: 32 layers, 1 full-attention layer then 3 sliding-window
    (2048) layers, repeated, over 4 sequences of 32768 tokens in a 65536-page pool."""
    _, pr, pool = bench.cfg4_pass(KvCache)
    windows = [0 if l % 4 == 0 else 2048 for l in range(32)]
    kv = hip.new_kv(32, pool, PAGE, HKV, D)
    try:
        bench._fill_arena(hip, kv, 32, bench.SEED + 41)
        _step(hip, kv, pr.meta, windows, bench.SEED + 42)
    finally:
        kv.destroy()


class _Both:
    """The product allocator and the allocator oracle driven through the same
    operations; every answer is compared before it is used."""

    def __init__(self, pool):
        self.a = KvCache(pool, 1 << 20, PAGE)
        self.b = OracleKvCache(pool, 1 << 20, PAGE)
        self.ids = {}  # product id -> oracle id

    def new_seq(self):
        s, t = self.a.new_seq(), self.b.new_seq()
        assert int(s) == int(t)
        self.ids[int(s)] = t
        return s

    def append(self, items):
        ca, cb = [], []
        pr = self.a.append([(s, toks) for s, toks in items], ca)
        want = self.b.append([(self.ids[int(s)], toks) for s, toks in items], cb)
        m = pr.meta
        got = (list(map(int, m.ids)), list(map(int, m.pos)), list(map(int, m.kv_slot)),
               list(map(int, m.pt_off)), list(map(int, m.pages)), pr.last)
        assert got == tuple(want), "pass metadata differs from the allocator oracle"
        assert [(c.src, c.dst) for c in ca] == cb
        return pr, ca

    def fork(self, s, n):
        ca, cb = [], []
        f = self.a.fork(s, n, ca)
        g = self.b.fork(self.ids[int(s)], n, cb)
        assert int(f) == int(g)
        self.ids[int(f)] = g
        assert [(c.src, c.dst) for c in ca] == cb, "fork copies differ from the allocator oracle"
        return f, ca

    def truncate(self, s, n):
        self.a.truncate(s, n)
        self.b.truncate(self.ids[int(s)], n)

    def free_seq(self, s):
        self.a.free_seq(s)
        self.b.free_seq(self.ids[int(s)])

    def check(self, seqs):
        for s in seqs:
            t = self.ids[int(s)]
            assert self.a.seq_len(s) == self.b.seq_len(t)
            assert list(self.a.seq_pages(s)) == list(self.b.seq_pages(t)), f"page table of {int(s)}"
        assert self.a.free_pages() == self.b.free_pages()


def test_cfg5_verify_fork_rollback_decode(hip):
    """cfg5 in full: 16 requests of ctx 4096 (2048 shared) verify 5 draft tokens; 8 of
    them fork 3 tokens back (inside the partly filled tail page: copy on write of that
    page, in every layer); all 24 roll back a seeded count in [0, 5]; then one decode
    step appends a token to each of the 24 sequences. All 24 layers of the configuration
    (distinct arenas): the copy-on-write page copy is checked in every layer, and the
    verify and the decode step after the rollback are checked against the oracle in
    every layer."""
    layers, pool = 24, 8192
    kv_ = _Both(pool)
    # The benchmark's scatter of the pool (bench._scatter), on both allocators.
    holders = [kv_.new_seq() for _ in range(pool)]
    for s in holders:
        kv_.append([(s, [0] * PAGE)])
    for i in permutation(pool, bench.SEED + 5):
        kv_.free_seq(holders[int(i)])
    base = kv_.new_seq()
    kv_.append([(base, [1] * 2048)])
    seqs = [kv_.fork(base, 2048)[0] for _ in range(16)]
    for s in seqs:
        kv_.append([(s, [1] * (4096 - 2048 - 5))])
    pr, cp = kv_.append([(s, [2] * 5) for s in seqs])
    assert not cp
    kv = hip.new_kv(layers, pool, PAGE, HKV, D)
    try:
        bench._fill_arena(hip, kv, layers, bench.SEED + 51)
        _step(hip, kv, pr.meta, [0] * layers, bench.SEED + 52)
        # Forks 3 tokens back: position 4093 lies inside the tail page (4096 tokens fill
        # 256 pages; 4093 = 255 * 16 + 13), so each fork copies that page.
        forks, copies = [], []
        for s in seqs[:8]:
            f, c = kv_.fork(s, kv_.a.seq_len(s) - 3)
            assert len(c) == 1, "a fork inside a partly filled page copies it"
            forks.append(f)
            copies += c
        src = np.array([c.src for c in copies], np.uint32)
        dst = np.array([c.dst for c in copies], np.uint32)
        assert len(set(dst.tolist())) == len(dst)
        hip.copy_pages(kv, copies)
        for l in range(layers):
            ks, vs = kv.read_pages(l, src)
            kd, vd = kv.read_pages(l, dst)
            assert np.array_equal(ks, kd) and np.array_equal(vs, vd), f"copied page bytes, layer {l}"
        back = uniform_ints(len(seqs) + len(forks), 0, 5, bench.SEED + 55)
        for s, n in zip(seqs + forks, back):
            kv_.truncate(s, kv_.a.seq_len(s) - int(n))
        kv_.check(seqs + forks)
        # The decode step after the rollback: one token on every sequence.
        pr2, cp2 = kv_.append([(s, [3]) for s in seqs + forks])
        hip.copy_pages(kv, cp2)
        kv_.check(seqs + forks)
        _step(hip, kv, pr2.meta, [0] * layers, bench.SEED + 53)
    finally:
        kv.destroy()
