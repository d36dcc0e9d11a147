"""Shared-prefix (cascade) decode: consecutive groups whose page tables start with the
same pages (forks of one sequence, kv.rs:277-295) read those keys once, as one group of
all their rows, and each group's merge takes that partial result first and its own
chunks after. Checked against the oracle with the cascade on and off, bit-reproducible,
through the fused append and through Backend::attention in one launch."""

import numpy as np
import pytest

from tests.scenario import D, Scenario, close

pytestmark = pytest.mark.gpu


def _option(hip, key, value):
    class _Ctx:
        def __enter__(self):
            hip.set_option(key, value)

        def __exit__(self, *a):
            hip.set_option(key, 1 if key == "attn_cascade" else 0)
    return _Ctx()


def _forks(sc, prefix, suffixes):
    """A base sequence of `prefix` tokens and one fork per suffix length; the forks'
    copy-on-write tail pages are copied on both sides."""
    base = sc.cache.new_seq()
    sc.prefill({base: prefix})
    seqs = []
    for _ in suffixes:
        copies = []
        seqs.append(sc.cache.fork(base, prefix, copies))
        sc.hip.copy_pages(sc.kv, copies)
        for c in copies:
            for o in sc.orc:
                o.copy_page(c.src, c.dst)
    sc.prefill({s: n for s, n in zip(seqs, suffixes) if n})
    return base, seqs


@pytest.mark.parametrize("hq,hkv", [(16, 4), (8, 4), (16, 2), (4, 4)])
@pytest.mark.parametrize("page,prefix", [(16, 600), (64, 1000), (16, 256)])
def test_shared_prefix_decode(hip, hq, hkv, page, prefix):
    sc = Scenario(hip, pages=9000 // page + 64, page=page, hkv=hkv, pool_seed=31)
    suffixes = [300, 0, 17, 1200, 5, 64, 999, 1]
    _, seqs = _forks(sc, prefix, suffixes)
    pr = sc.run_pass([(s, 1) for s in seqs])
    rows = len(pr.meta.pos)
    kk = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    vv = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    got = hip.attend_append(sc.kv, 0, kk, vv, q, hq)  # fused append + cascade
    sc.orc[0].store(pr.meta.kv_slot, kk.reshape(rows, -1), vv.reshape(rows, -1))
    again = hip.attend(sc.kv, 0, q, hq)
    with _option(hip, "attn_cascade", 0):
        plain = hip.attend(sc.kv, 0, q, hq)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    for name, a in (("cascade", got), ("again", again), ("plain", plain)):
        assert close(a, want).all(), f"{name}: max abs err {np.abs(a - want).max()}"
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    exact = sc.orc[0].attend_f64(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert np.abs(got - exact).max() < 2e-5


@pytest.mark.parametrize("target_waves", [0, 4096])
@pytest.mark.parametrize("k,window", [(2, 0), (1, 5000), (1, 700)])
def test_shared_prefix_chunks_rows_and_windows(hip, target_waves, k, window):
    """Many chunks per group (the merge's range split over the prefix's and own
    chunks), two rows per sequence, a window that cuts nothing (cascade) and one that
    cuts the prefix (no cascade)."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=700, page=16, hkv=hkv, pool_seed=32)
    _, seqs = _forks(sc, 2000, [100, 2500, 40, 900])
    pr = sc.run_pass([(s, k) for s in seqs])
    sc.store(pr)
    rows = len(pr.meta.pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    with _option(hip, "attn_target_waves", target_waves):
        got = hip.attend(sc.kv, 0, q, hq, window=window)
        again = hip.attend(sc.kv, 0, q, hq, window=window)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_shared_prefix_backend_attention_in_one_launch(hip):
    """Backend::attention with the rows' write_rows in the same launch gives the bits of
    write_rows then attention as two calls, with the cascade in both."""
    from yaxus_amd.rope import inv_freq, rope_table

    hq, hkv = 16, 4
    f = inv_freq(D, 10000.0)
    table = rope_table(f, 1.0, 4096)
    outs = []
    for one_launch in (True, False):
        sc = Scenario(hip, pages=400, page=16, hkv=hkv, pool_seed=33)
        _, seqs = _forks(sc, 700, [50, 300, 0, 800])
        pr = sc.run_pass([(s, 1) for s in seqs])
        rows = len(pr.meta.pos)
        qkv = sc.draw(rows * (hq + 2 * hkv) * D).reshape(rows, -1)
        qn, kn = sc.draw(D) * 0.1, sc.draw(D) * 0.1
        if one_launch:
            got = hip.attention(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
        else:
            qq = hip.qk_rope_append(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
            got = hip.attend(sc.kv, 0, qq, hq)
        outs.append(got)
        if not one_launch:
            want = sc.orc[0]
            qo = want.write_rows(qkv, hq, qn, kn, 1e-6, f, 1.0, pr.meta.pos, pr.meta.kv_slot)
            ref = want.attend(qo, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
            assert close(got, ref).all(), f"max abs err {np.abs(got - ref).max()}"
        sc.kv.destroy()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_shared_prefix_f32_arena(hip):
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=400, page=16, hkv=hkv, pool_seed=34, f32=True)
    _, seqs = _forks(sc, 900, [10, 400, 77, 1])
    pr = sc.run_pass([(s, 1) for s in seqs])
    sc.store(pr)
    rows = len(pr.meta.pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    got = hip.attend(sc.kv, 0, q, hq)
    exact = sc.orc[0].attend_f64(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert np.abs(got - exact).max() < 1e-5


@pytest.mark.parametrize("cut", [1, 7, 14])
def test_shared_prefix_window_cutting_inside_the_first_block(hip, cut):
    """A window that leaves every row's first visible key inside block 0 (1-15 keys cut):
    the rows still start at block 0, so the shared prefix is attended once for all of
    them, and each row's window mask applies inside the shared blocks. The rows' positions
    differ by at most one, so every row's cut stays within 1-15."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=700, page=16, hkv=hkv, pool_seed=35)
    _, seqs = _forks(sc, 2000, [40, 41, 40, 41])
    pr = sc.run_pass([(s, 1) for s in seqs])
    sc.store(pr)
    rows = len(pr.meta.pos)
    pos = np.asarray(pr.meta.pos)
    window = int(pos.min()) + 1 - cut  # the earliest row sees keys from `cut` on
    assert all(0 < p + 1 - window < 16 for p in pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    got = hip.attend(sc.kv, 0, q, hq, window=window)
    with _option(hip, "attn_cascade", 0):
        plain = hip.attend(sc.kv, 0, q, hq, window=window)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    for name, a in (("cascade", got), ("plain", plain)):
        assert close(a, want).all(), f"{name}: max abs err {np.abs(a - want).max()}"
    # The window matters: attention over the whole prefix differs.
    full = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert np.abs(full - want).max() > 1e-6
