"""The benchmark configurations at their full sizes, every row against the oracle.

The passes are the benchmark's own (bench.py's builders over the product allocator);
the arena is filled on the device (yx_fill_normal), the rows' q/k/v are seeded N(0,1)
on the host. After the product call, the pages the pass reads are copied back into the
oracle's slot-major arena, so the oracle attends over the same K/V bits; the appended
K/V are checked separately against their binary16 roundings, bit for bit, so a wrong
append cannot hide behind the mirrored arena.
"""

import os

import numpy as np
import pytest

import bench
from oracle.attn import OracleArena, f32_to_f16_bits, normal
from tests.scenario import close
from yaxus_amd import KvCache

pytestmark = pytest.mark.gpu
D, HQ, HKV, PAGE = bench.D, bench.HQ, bench.HKV, bench.PAGE
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _mirror(orc, kv, pages):
    """Copies the device pages into the oracle arena (device order [hkv][page][d] to
    slot-major [slot][hkv * d])."""
    pages = np.unique(np.asarray(pages, np.uint32))
    for part in np.array_split(pages, max(1, len(pages) // 2048)):
        k, v = kv.read_pages(0, part)
        slots = (part.astype(np.int64)[:, None] * PAGE + np.arange(PAGE)).reshape(-1)
        orc.k[slots] = k.transpose(0, 2, 1, 3).reshape(len(part) * PAGE, HKV * D)
        orc.v[slots] = v.transpose(0, 2, 1, 3).reshape(len(part) * PAGE, HKV * D)


def _run(hip, pr, pool, seed, windows=(0,)):
    """Fused append + attention of the pass on a filled one-layer arena, then each
    window's attention again; returns (outputs per window, oracle outputs)."""
    rows = len(pr.meta.pos)
    kv = hip.new_kv(1, pool, PAGE, HKV, D)
    try:
        bench._fill_arena(hip, kv, 1, seed)
        k = normal(rows * HKV * D, seed + 1, 0).reshape(rows, HKV, D)
        v = normal(rows * HKV * D, seed + 2, 0).reshape(rows, HKV, D)
        q = normal(rows * HQ * D, seed + 3, 0).reshape(rows, HQ * D)
        hip.begin_pass(pr.meta)
        got = [hip.attend_append(kv, 0, k, v, q, HQ, window=windows[0])]
        for w in windows[1:]:
            got.append(hip.attend(kv, 0, q, HQ, window=w))
        # The appended K/V, bit for bit.
        slots = np.asarray(pr.meta.kv_slot, np.int64)
        kk, vv = kv.read_pages(0, np.unique(slots // PAGE).astype(np.uint32))
        index = {int(p): i for i, p in enumerate(np.unique(slots // PAGE))}
        for r, s in enumerate(slots):
            i, off = index[int(s // PAGE)], int(s % PAGE)
            assert np.array_equal(kk[i, :, off, :], f32_to_f16_bits(k[r])), f"K of row {r}"
            assert np.array_equal(vv[i, :, off, :], f32_to_f16_bits(v[r])), f"V of row {r}"
        orc = OracleArena(pool, PAGE, HKV, D, f16=True)
        _mirror(orc, kv, pr.meta.pages)
    finally:
        kv.destroy()
    want = [orc.attend(q, HQ, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=w, threads=THREADS)
            for w in windows]
    return got, want, (orc, q)


def _check(got, want, what):
    for g, w in zip(got, want):
        assert close(g, w).all(), f"{what}: max abs err {np.abs(g - w).max()}"


def test_headline_b16_ctx4096(hip):
    """B=16, ctx 4096 (4095 prior + 1 appended), pages scattered over 8192."""
    _, pr = bench.build_pass(KvCache)
    got, want, (orc, q) = _run(hip, pr, bench.POOL, bench.SEED + 11)
    _check(got, want, "headline")
    exact = orc.attend_f64(q, HQ, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert np.abs(got[0] - exact).max() < 2e-5


def test_cfg2_prefix_sharing(hip):
    """16 requests on one shared 1024-token prefix plus suffixes U[512, 3072]."""
    _, pr, pool, _ = bench.cfg2_pass(KvCache)
    got, want, _ = _run(hip, pr, pool, bench.SEED + 12)
    _check(got, want, "cfg2")


def test_cfg3_chunked_prefill(hip):
    """16 chunks of 256 rows (4096 rows) on contexts U[0, 2048]: the prefill kernel."""
    _, pr, pool, _ = bench.cfg3_pass(KvCache)
    got, want, _ = _run(hip, pr, pool, bench.SEED + 13)
    _check(got, want, "cfg3")


def test_cfg4_long_context_full_and_window(hip):
    """4 requests of 32768 tokens over a 65536-page pool: a full layer and a window-2048
    layer on the same K/V."""
    _, pr, pool = bench.cfg4_pass(KvCache)
    got, want, _ = _run(hip, pr, pool, bench.SEED + 14, windows=(0, 2048))
    _check(got, want, "cfg4")


def test_cfg5_verify(hip):
    """16 requests of ctx 4096 (2048 shared) verifying 5 rows each."""
    _, pr, pool, _ = bench.cfg5_pass(KvCache)
    got, want, _ = _run(hip, pr, pool, bench.SEED + 15)
    _check(got, want, "cfg5")
