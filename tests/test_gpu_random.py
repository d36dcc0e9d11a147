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


@pytest.mark.parametrize("seed", range(24))
def test_random_forked_pass_matches_oracle(hip, seed):
    """Random forks of one or two prompts (shared whole pages, copied tails) mixed with
    unrelated sequences, in random pass order: the shared-prefix path where it applies."""
    rng = np.random.default_rng(7000 + seed)
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    page = PAGES[rng.integers(4)]
    prompts = [int(x) for x in rng.integers(page, 1400, int(rng.integers(1, 3)))]
    nfork = [int(x) for x in rng.integers(2, 7, len(prompts))]
    suffix = [[int(x) for x in rng.integers(0, 500, n)] for n in nfork]
    loners = [int(x) for x in rng.integers(0, 900, int(rng.integers(0, 3)))]
    rows = int(rng.choice([1, 1, 2]))
    mixed = bool(rng.integers(2))  # rows per sequence drawn per sequence (1 or 2)
    window = 0 if rng.integers(3) else int(rng.integers(200, 3000))
    need = sum((p + page - 1) // page for p in prompts) + sum(
        (p + s + rows + page - 1) // page + 1 for p, ss in zip(prompts, suffix) for s in ss) + sum(
        (n + rows + page - 1) // page for n in loners)
    sc = Scenario(hip, pages=need + 8, page=page, hkv=hkv, pool_seed=seed)
    try:
        seqs = []
        for p, ss in zip(prompts, suffix):
            base = sc.cache.new_seq()
            sc.prefill({base: p})
            for s in ss:
                copies = []
                f = sc.cache.fork(base, p, copies)
                sc.hip.copy_pages(sc.kv, copies)
                for c in copies:
                    sc.orc[0].copy_page(c.src, c.dst)
                if s:
                    sc.prefill({f: s})
                seqs.append(f)
        for n in loners:
            s = sc.cache.new_seq()
            if n:
                sc.prefill({s: n})
            seqs.append(s)
        order = [seqs[i] for i in rng.permutation(len(seqs))] if rng.integers(2) else seqs
        pr = sc.run_pass([(s, int(rng.integers(1, 3)) if mixed else rows) for s in order])
        n = len(pr.meta.pos)
        k = sc.draw(n * hkv * D).reshape(n, hkv, D)
        v = sc.draw(n * hkv * D).reshape(n, hkv, D)
        q = sc.draw(n * hq * D).reshape(n, hq * D)
        got = sc.hip.attend_append(sc.kv, 0, k, v, q, hq, window=window)
        sc.orc[0].store(pr.meta.kv_slot, k.reshape(n, -1), v.reshape(n, -1))
        want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
        case = f"heads {hq}/{hkv} page {page} prompts {prompts} suffix {suffix} rows {rows} mixed {mixed} window {window}"
        assert close(got, want).all(), f"{case}: max abs err {np.abs(got - want).max()}"
    finally:
        sc.kv.destroy()
