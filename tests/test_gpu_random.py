"""Seeded random passes through the fused append + attention against the oracle: head
shapes, page sizes (16-512), sequence counts, context lengths, rows per sequence
(decode, verify and prefill rows mixed in one pass) and windows drawn per case. Each
case also checks the appended K/V bits of every page the pass wrote."""

import numpy as np
import pytest

from tests.scenario import D, Scenario, close

pytestmark = pytest.mark.gpu

HEADS = [(16, 4), (8, 8), (32, 2), (16, 1), (8, 2), (4, 4), (12, 4), (10, 2), (14, 2), (6, 1)]
PAGES = [16, 32, 64, 128, 256, 512]
ROWS = [1, 1, 1, 2, 5, 40]


@pytest.mark.parametrize("seed", range(48))
def test_random_pass_matches_oracle(hip, seed):
    rng = np.random.default_rng(9000 + seed)
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    page = PAGES[rng.integers(len(PAGES))]
    nseq = int(rng.integers(1, 9))
    prior = [int(x) for x in rng.integers(0, 1500, nseq)]
    rows = [ROWS[rng.integers(len(ROWS))] for _ in range(nseq)]
    window = 0 if rng.integers(2) == 0 else int(rng.integers(1, 600))
    need = sum((p + r + page - 1) // page for p, r in zip(prior, rows))
    sc = Scenario(hip, pages=need + 8, page=page, hkv=hkv, pool_seed=seed)
    try:
        seqs = [sc.cache.new_seq() for _ in range(nseq)]
        sc.prefill({s: n for s, n in zip(seqs, prior) if n})
        pr = sc.run_pass(list(zip(seqs, rows)))
        n = len(pr.meta.pos)
        k = sc.draw(n * hkv * D).reshape(n, hkv, D)
        v = sc.draw(n * hkv * D).reshape(n, hkv, D)
        q = sc.draw(n * hq * D).reshape(n, hq * D)
        got = sc.hip.attend_append(sc.kv, 0, k, v, q, hq, window=window)
        sc.orc[0].store(pr.meta.kv_slot, k.reshape(n, -1), v.reshape(n, -1))
        want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
        case = f"heads {hq}/{hkv} page {page} prior {prior} rows {rows} window {window}"
        assert close(got, want).all(), f"{case}: max abs err {np.abs(got - want).max()}"
        written = sorted({int(s) // page for s in pr.meta.kv_slot})
        kk, vv = sc.kv.read_pages(0, np.array(written, np.uint32))
        for i, p in enumerate(written):
            ok, ov = sc.orc[0].page_bits(p)
            assert np.array_equal(kk[i], ok) and np.array_equal(vv[i], ov), f"{case}: page {p}"
    finally:
        sc.kv.destroy()
