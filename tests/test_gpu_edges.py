"""Edge cases of the device path against the oracle: windows of 1 key and windows that
cover exactly the context, rows at position 0, appends that open a new page, passes
with no rows, and a pass whose sequences have very different lengths. Decode, verify
and prefill shapes each, through the fused append + attention."""

import numpy as np
import pytest

from tests.scenario import D, Scenario, close

pytestmark = pytest.mark.gpu


def _run(hip, hq, hkv, page, prior, rows, window, seed):
    sc = Scenario(hip, pages=sum((p + r + page - 1) // page for p, r in zip(prior, rows)) + 4,
                  page=page, hkv=hkv, pool_seed=seed)
    try:
        seqs = [sc.cache.new_seq() for _ in prior]
        sc.prefill({s: n for s, n in zip(seqs, prior) if n})
        pr = sc.run_pass(list(zip(seqs, rows)))
        n = len(pr.meta.pos)
        k = sc.draw(n * hkv * D).reshape(n, hkv, D)
        v = sc.draw(n * hkv * D).reshape(n, hkv, D)
        q = sc.draw(n * hq * D).reshape(n, hq * D)
        got = hip.attend_append(sc.kv, 0, k, v, q, hq, window=window)
        sc.orc[0].store(pr.meta.kv_slot, k.reshape(n, -1), v.reshape(n, -1))
        want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
        assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
        return got, v, pr
    finally:
        sc.kv.destroy()


@pytest.mark.parametrize("rows", [1, 5, 40])
def test_window_of_one_key_returns_the_rows_own_value(hip, rows):
    """window 1: each row sees only its own key, so the output is its own V (per KV head)."""
    hq, hkv = 8, 2
    got, v, _ = _run(hip, hq, hkv, 16, [37, 300, 0], [rows] * 3, 1, 31)
    want = np.repeat(v.astype(np.float16).astype(np.float32), hq // hkv, axis=1).reshape(got.shape)
    assert np.abs(got - want).max() < 2e-3


@pytest.mark.parametrize("rows", [1, 5, 40])
def test_window_equal_to_the_context_is_full_attention(hip, rows):
    """A window exactly as long as the longest context changes nothing."""
    prior = [15, 100, 31]
    w = max(prior) + rows
    a, _, _ = _run(hip, 16, 4, 16, prior, [rows] * 3, w, 32)
    b, _, _ = _run(hip, 16, 4, 16, prior, [rows] * 3, 0, 32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("page", [16, 64])
def test_first_rows_and_page_boundaries(hip, page):
    """Sequences starting at position 0, and appends that open a new page (prior a
    multiple of the page size) or end one (prior + rows a multiple)."""
    prior = [0, page, 2 * page - 1, 3 * page - 5]
    _run(hip, 16, 4, page, prior, [1, 1, 1, 5], 0, 33)
    _run(hip, 16, 4, page, prior, [40, 40, 40, 40], 0, 34)


def test_lengths_far_apart_in_one_pass(hip):
    """One sequence of a few keys next to one of thousands, decode and verify."""
    _run(hip, 16, 4, 16, [3, 6000], [1, 1], 0, 35)
    _run(hip, 16, 4, 16, [3, 6000], [5, 5], 0, 36)
    _run(hip, 16, 4, 16, [3, 6000], [40, 1], 0, 37)


def test_a_pass_with_no_rows(hip):
    """No rows: every call is a no-op that returns at once."""
    sc = Scenario(hip, pages=8, page=16, hkv=2, pool_seed=38)
    try:
        pr = sc.run_pass([])
        assert len(pr.meta.pos) == 0
        out = hip.attend(sc.kv, 0, np.zeros((0, 8 * D), np.float32), 8)
        assert out.shape[0] == 0
        hip.sync()
    finally:
        sc.kv.destroy()
