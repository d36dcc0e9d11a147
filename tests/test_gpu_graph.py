"""HIP-graph replay of the attention launches (how bench.py times them, and how an
engine would replay a step): every replay gives the eager call's bits, with eager
launches and synchronisations of the program between the replays. The split-K arrival
counters are left at zero by the kernels themselves, so no memset is captured."""

import numpy as np
import pytest

from tests.scenario import D, Scenario

pytestmark = pytest.mark.gpu


def _forks(sc, prefix, suffixes):
    base = sc.cache.new_seq()
    sc.prefill({base: prefix})
    seqs = []
    for _ in suffixes:
        copies = []
        seqs.append(sc.cache.fork(base, prefix, copies))
        sc.hip.copy_pages(sc.kv, copies)
    sc.prefill({s: n for s, n in zip(seqs, suffixes) if n})
    return seqs


def _case(hip, kind):
    hkv = 4
    f32 = kind == "f32"
    sc = Scenario(hip, pages=800, page=16, hkv=hkv, pool_seed=41, layers=2, f32=f32)
    if kind == "cascade":
        seqs = _forks(sc, 1200, [100, 900, 30, 2000])
        k = 1
    else:
        seqs = [sc.cache.new_seq() for _ in range(5)]
        sc.prefill(dict(zip(seqs, [4095, 1000, 17, 2500, 300])))
        k = {"decode": 1, "verify": 5, "prefill": 64, "f32": 1}[kind]
    pr = sc.run_pass([(s, k) for s in seqs])
    return sc, pr


@pytest.mark.parametrize("kind", ["decode", "cascade", "verify", "prefill", "f32"])
def test_graph_replays_match_eager(hip, kind):
    hq = 16
    sc, pr = _case(hip, kind)
    rows = len(pr.meta.pos)
    hkv = sc.hkv
    q = hip.tensor((rows, hq * D))
    k = hip.tensor((rows, hkv * D))
    v = hip.tensor((rows, hkv * D))
    outs = [hip.tensor((rows, hq * D)) for _ in range(2)]
    for i, t in enumerate((q, k, v)):
        hip.fill_normal(t.ptr, t.nbytes // 4, False, 77, i << 32)

    def step():
        hip.attend_append(sc.kv, 0, k, v, q, hq, out=outs[0])
        hip.attend(sc.kv, 1, q, hq, window=700, out=outs[1])

    step()
    hip.sync()
    eager = [o.numpy() for o in outs]
    hip.graph_begin()
    step()
    hip.graph_end()
    for rep in range(3):
        for o in outs:
            hip.fill_normal(o.ptr, o.nbytes // 4, False, 99, rep << 32)  # eager work between
        hip.sync()
        hip.graph_launch()
        hip.sync()
        for i, o in enumerate(outs):
            got = o.numpy()
            assert np.array_equal(got.view(np.uint32), eager[i].view(np.uint32)), f"replay {rep}, layer {i}"
        step()  # an eager step between replays as well
        hip.sync()
    for t in (q, k, v, *outs):
        t.free()
    sc.kv.destroy()
