"""The entry point that allocates nothing (yx_attention_append_noalloc) against the one it
varies (yx_attention_append_dev): the same kernels over the library's static scratch, so
the outputs must be the same bits. Two passes in a row, the second smaller than the
first, then a prefill pass and a repeat of a pass (the scratch keeps the previous call's
contents; the arrival counters must be back at zero); and a pass too large for the
scratch is refused with a status, not run."""

import ctypes

import numpy as np
import pytest

from tests.scenario import D, Scenario
from yaxus_amd._lib import check_hip

pytestmark = pytest.mark.gpu
HQ, HKV = 16, 4
YX_ERR_UNSUPPORTED = 6  # include/yaxus_kv_cache.h


def _inputs(hip, sc, rows, seed):
    k = sc.draw(rows * HKV * D).reshape(rows, HKV, D)
    v = sc.draw(rows * HKV * D).reshape(rows, HKV, D)
    q = sc.draw(rows * HQ * D).reshape(rows, HQ * D)
    return [hip.tensor(a.shape).upload(a) for a in (k, v, q)]


def _both(hip, sc, rows, window=0):
    """Out of the regular entry point and of the no-alloc one on the same inputs (the
    append stores the same bits both times)."""
    k, v, q = _inputs(hip, sc, rows, 0)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    outs = []
    try:
        for fn in (hip.L.yx_attention_append_dev, hip.L.yx_attention_append_noalloc,
                   hip.L.yx_attention_append_noalloc):
            o = hip.tensor((rows, HQ * D))
            check_hip(fn(hip.ctx, sc.kv.h, 0, k.ptr, v.ptr, q.ptr, o.ptr, HQ, HKV, window, scale))
            outs.append(o.numpy())
            o.free()
    finally:
        for t in (k, v, q):
            t.free()
    return outs


def test_no_alloc_entry_point_matches_the_allocating_one(hip):
    sc = Scenario(hip, pages=3072, page=16, hkv=HKV, pool_seed=7, seed=99)
    try:
        seqs = [sc.cache.new_seq() for _ in range(12)]
        sc.prefill(dict(zip(seqs, [3000, 2500, 4000, 1200, 3900, 2048, 777, 3333, 64, 2999, 3500, 1800])),
                   chunk=4096)
        # 1: a decode pass of 12 sequences (split-K: partials and counters in use).
        sc.run_pass([(s, 1) for s in seqs])
        a, b, b2 = _both(hip, sc, 12)
        assert np.array_equal(a, b) and np.array_equal(b, b2)
        # 2: a smaller pass, verify rows of 3 sequences, with a window.
        sc.run_pass([(s, 5) for s in seqs[:3]])
        a, b, b2 = _both(hip, sc, 15, window=700)
        assert np.array_equal(a, b) and np.array_equal(b, b2)
        # 3: a prefill pass (the prefill kernel's work list in the scratch).
        sc.run_pass([(seqs[4], 96)])
        a, b, b2 = _both(hip, sc, 96)
        assert np.array_equal(a, b) and np.array_equal(b, b2)
        # 4: the first shape again after the others.
        sc.run_pass([(s, 1) for s in seqs])
        a, b, b2 = _both(hip, sc, 12)
        assert np.array_equal(a, b) and np.array_equal(b, b2)
    finally:
        sc.kv.destroy()


def test_no_alloc_refuses_a_pass_beyond_the_scratch(hip):
    sc = Scenario(hip, pages=4200, page=16, hkv=HKV, pool_seed=8, seed=5)
    try:
        seqs = [sc.cache.new_seq() for _ in range(16)]
        sc.prefill({s: 4095 for s in seqs}, chunk=8192)
        sc.run_pass([(s, 1) for s in seqs])
        # Chunks of 4 blocks: 64 per group, 4 MiB of partials per kv head.
        hip.set_option("attn_target_waves", 1 << 20)
        hip.set_option("attn_max_chunk_blocks", 4)
        k, v, q = _inputs(hip, sc, 16, 0)
        o = hip.tensor((16, HQ * D))
        try:
            scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
            rc = hip.L.yx_attention_append_noalloc(hip.ctx, sc.kv.h, 0, k.ptr, v.ptr, q.ptr, o.ptr,
                                                   HQ, HKV, 0, scale)
            assert rc == YX_ERR_UNSUPPORTED
            assert b"scratch" in hip.L.yx_last_error()
            # The allocating entry point runs the same pass.
            check_hip(hip.L.yx_attention_append_dev(hip.ctx, sc.kv.h, 0, k.ptr, v.ptr, q.ptr, o.ptr,
                                                    HQ, HKV, 0, scale))
            hip.sync()
        finally:
            hip.set_option("attn_target_waves", 0)
            hip.set_option("attn_max_chunk_blocks", 1 << 20)
            for t in (k, v, q, o):
                t.free()
    finally:
        sc.kv.destroy()
