"""The entry point that allocates nothing (yx_attention_append_noalloc) against the one it
varies (yx_attention_append_dev): the same kernels over the library's static scratch, so
the outputs must be the same bits. Two passes in a row, the second smaller than the
first, then a prefill pass and a repeat of a pass (the scratch keeps the previous call's
contents; the arrival counters must be back at zero); a decode step's pattern, one call
per layer over 32 layers of alternating window and full attention, in a pass whose work
lists go to the scratch and in the next one (whose lists yx_pass_begin prebuilt), with a
second context taking the scratch over between calls; and a pass too large for the
scratch is refused with a status, not run."""

import ctypes

import numpy as np
import pytest

from tests.scenario import D, Scenario
from yaxus_amd._lib import check_hip

pytestmark = pytest.mark.gpu
HQ, HKV = 16, 4
YX_ERR_UNSUPPORTED = 6  # include/yaxus_kv_cache.h


def _inputs(hip, sc, rows, seed=0):
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


def _call(hip, sc, fn, layer, rows, window, ins):
    k, v, q = ins
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o = hip.tensor((rows, HQ * D))
    try:
        check_hip(fn(hip.ctx, sc.kv.h, layer, k.ptr, v.ptr, q.ptr, o.ptr, HQ, HKV, window, scale))
        return o.numpy()
    finally:
        o.free()


def test_no_alloc_once_per_layer_over_32_layers(hip):
    """A decode loop's pattern: one no-alloc call per layer, 32 layers (window 256 on odd
    layers, full attention on even ones: two work lists per pass), over two passes. The
    first pass's lists are sent to the scratch's list region (once per list, not per
    call); the second pass's were prebuilt by yx_pass_begin. Every output equals the
    allocating entry point's bit for bit. Between layers a second context on the same GPU
    runs its own no-alloc call, so the scratch changes hands both ways."""
    from yaxus_amd.backend import HipBackend

    L = 32
    sc = Scenario(hip, pages=640, page=16, hkv=HKV, layers=L, pool_seed=11, seed=31)
    hip2 = HipBackend(0)
    sc2 = Scenario(hip2, pages=256, page=16, hkv=HKV, pool_seed=12, seed=32)
    try:
        seqs = [sc.cache.new_seq() for _ in range(8)]
        sc.prefill(dict(zip(seqs, [1200, 900, 1500, 333, 1024, 700, 1111, 64])), chunk=4096)
        s2 = [sc2.cache.new_seq() for _ in range(3)]
        sc2.prefill(dict(zip(s2, [1000, 700, 900])), chunk=4096)
        sc2.run_pass([(s, 1) for s in s2])
        for step in range(2):
            sc.run_pass([(s, 1) for s in seqs])
            for layer in range(L):
                window = 256 if layer % 2 else 0
                ins = _inputs(hip, sc, 8)
                try:
                    # The no-alloc call first, so that in the first pass its list is not
                    # on the device yet.
                    b = _call(hip, sc, hip.L.yx_attention_append_noalloc, layer, 8, window, ins)
                    a = _call(hip, sc, hip.L.yx_attention_append_dev, layer, 8, window, ins)
                    assert np.array_equal(a, b), f"step {step} layer {layer}"
                    if layer % 8 == 3:
                        ins2 = _inputs(hip2, sc2, 3)
                        try:
                            b2 = _call(hip2, sc2, hip2.L.yx_attention_append_noalloc, 0, 3, 0, ins2)
                            a2 = _call(hip2, sc2, hip2.L.yx_attention_append_dev, 0, 3, 0, ins2)
                        finally:
                            for t in ins2:
                                t.free()
                        assert np.array_equal(a2, b2), f"second context, step {step} layer {layer}"
                finally:
                    for t in ins:
                        t.free()
    finally:
        sc2.kv.destroy()
        hip2.close()
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
