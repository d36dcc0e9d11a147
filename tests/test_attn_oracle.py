"""Pins the attention oracle (oracle/attn_oracle.c) before it is trusted as a checker.

- binary16 rounding vs numpy's IEEE-754 conversion at every f16 boundary, tie and
  subnormal, plus a strided sweep of all f32 bit patterns; all 65536 decodes;
- the 16-lane dot order (backend-cpu lib.rs:280-294) bit for bit;
- the reference test `paged_attention_matches_dense_attention` (backend-cpu
  lib.rs:676-714) restated with its xorshift values, vs an independent numpy dense
  attention (f64), bound 1e-5 as in the reference;
- closed forms: one key gives V; equal scores give the mean of V; a window at least
  the context is full attention; page placement does not change a bit; the f32
  two-pass result is within 1e-5 of an f64 brute force at context 4096.
"""

import numpy as np
import pytest

from oracle.attn import OracleArena, f32_to_f16_bits, lib

D = 128


def _f16_oracle(x):
    return f32_to_f16_bits(np.asarray(x, np.float32))


def _f16_numpy(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def test_f16_rounding_at_every_boundary():
    h = np.arange(0, 0x7C00, dtype=np.uint32)  # every finite non-negative f16
    v = h.astype(np.uint16).view(np.float16).astype(np.float32)
    nxt = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((v.astype(np.float64) + nxt) / 2).astype(np.float32)  # exact ties (f32 holds them)
    cands = [v, mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)),
             np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(0))]
    x = np.concatenate(cands + [-c for c in cands])
    assert np.array_equal(_f16_oracle(x), _f16_numpy(x))


def test_f16_rounding_over_all_exponents_and_specials():
    bits = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    a, b = _f16_oracle(x), _f16_numpy(x)
    nan = np.isnan(x)
    assert np.array_equal(a[~nan], b[~nan])
    # NaN stays NaN (payload bits are not part of the contract)
    assert np.all((a[nan] & 0x7C00) == 0x7C00) and np.all((a[nan] & 0x3FF) != 0)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.996, 65520, 2 ** -24,
                        2 ** -25, 2 ** -25 * 1.0000001, 2 ** -14, 2 ** -14 * (1 - 2 ** -11)],
                       np.float32)
    assert np.array_equal(_f16_oracle(special), _f16_numpy(special))


def test_f16_decode_is_exact():
    L = lib()
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([L.orc_f16_to_f32(int(i)) for i in h], np.float32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def _dot16(a, b):
    """lib.rs:280-294: 16 f32 accumulators over whole chunks, summed in order, then the rest."""
    acc = np.zeros(16, np.float32)
    n = len(a) // 16 * 16
    for c in range(0, n, 16):
        acc = (acc + a[c:c + 16] * b[c:c + 16]).astype(np.float32)
    s = np.float32(0)
    for i in range(16):
        s = np.float32(s + acc[i])
    for i in range(n, len(a)):
        s = np.float32(s + np.float32(a[i] * b[i]))
    return s


@pytest.mark.parametrize("n", [1, 8, 15, 16, 17, 128, 130])
def test_dot_follows_the_16_lane_order(n):
    import ctypes

    rng = np.random.default_rng(n)
    for _ in range(20):
        a = rng.standard_normal(n).astype(np.float32) * np.float32(rng.uniform(0.1, 1e3))
        b = rng.standard_normal(n).astype(np.float32)
        got = lib().orc_dot(a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p), n)
        assert np.float32(got).view(np.uint32) == _dot16(a, b).view(np.uint32)


def _values(n, seed):
    """backend-cpu lib.rs:572-582: small deterministic values in [-1, 1) (xorshift)."""
    M = (1 << 64) - 1
    s = ((seed * 0x9E3779B97F4A7C15) & M) | 1
    out = np.empty(n, np.float32)
    for i in range(n):
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        out[i] = np.float32(np.float32(s >> 40) / np.float32(1 << 23) - np.float32(1.0))
    return out


def _dense(qkv_rows, hq, hkv, d, inv_freq, conc, eps, window):
    """Dense attention of one sequence (positions 0..n), f64, from first principles:
    RMSNorm (weight 0, offset 1), half-split RoPE, causal softmax."""
    n = len(qkv_rows)
    x = np.asarray(qkv_rows, np.float64)
    qd, kvd = hq * d, hkv * d

    def norm(v):
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + eps)

    ang = np.arange(n)[:, None] * np.asarray(inv_freq, np.float64)[None, :]
    cs, sn = np.cos(ang) * conc, np.sin(ang) * conc

    def rope(v):  # v [n, heads, d]
        h = d // 2
        a, b = v[..., :h], v[..., h:]
        return np.concatenate([a * cs[:, None] - b * sn[:, None], b * cs[:, None] + a * sn[:, None]], -1)

    q = rope(norm(x[:, :qd].reshape(n, hq, d)))
    k = rope(norm(x[:, qd:qd + kvd].reshape(n, hkv, d)))
    v = x[:, qd + kvd:].reshape(n, hkv, d)
    out = np.zeros((n, hq, d))
    for p in range(n):
        lo = max(0, p + 1 - window) if window else 0
        for h in range(hq):
            kh = h // (hq // hkv)
            s = k[lo:p + 1, kh] @ q[p, h] / np.sqrt(d)
            w = np.exp(s - s.max())
            out[p, h] = (w[:, None] * v[lo:p + 1, kh]).sum(0) / w.sum()
    return out.reshape(n, qd)


@pytest.mark.parametrize("window", [None, 16])
def test_paged_attention_matches_dense_attention(window):
    """backend-cpu lib.rs:676-714 restated: two sequences on non-adjacent pages [3, 1]
    and [0], lengths 140 and 9, two passes crossing a page boundary, PAGE = 128."""
    hq, hkv, d, P, eps = 4, 2, 8, 128, 1e-6
    inv_freq, conc = np.array([1.0, 0.3, 0.05, 0.01], np.float32), np.float32(1.1)
    cols = (hq + 2 * hkv) * d
    pages = [[3, 1], [0]]
    lens = [140, 9]
    qkv = [[_values(cols, s * 1000 + p) for p in range(n)] for s, n in enumerate(lens)]
    want = [_dense(q, hq, hkv, d, inv_freq, conc, eps, window) for q in qkv]
    arena = OracleArena(4, P, hkv, d, f16=False)
    zero = np.zeros(d, np.float32)
    got = [np.zeros((n, hq * d), np.float32) for n in lens]
    first = [(0, p) for p in range(100)] + [(1, p) for p in range(4)]
    second = [(0, p) for p in range(100, 140)] + [(1, p) for p in range(4, 9)]
    for rows in (first, second):
        meta_pages, off = [], {}
        for sq, _ in rows:
            if sq not in off:
                off[sq] = len(meta_pages)
                meta_pages += pages[sq]
        pos = np.array([p for _, p in rows], np.uint32)
        slot = np.array([pages[s][p // P] * P + p % P for s, p in rows], np.uint32)
        pt_off = np.array([off[s] for s, _ in rows], np.uint32)
        x = np.stack([qkv[s][p] for s, p in rows])
        # write_rows groups rows by their cos/sin only through pos: one call per pass
        q = arena.write_rows(x, hq, zero, zero, eps, inv_freq, conc, pos, slot)
        o = arena.attend(q, hq, pos, pt_off, np.array(meta_pages, np.uint32), window=window or 0)
        for r, (s, p) in enumerate(rows):
            got[s][p] = o[r]
    for s in range(2):
        assert np.abs(got[s] - want[s]).max() < 1e-5


def _arena_with(keys, vals, page=16, hkv=1, pages_of=None, npages=None):
    n = len(keys)
    npg = -(-n // page)
    pt = np.arange(npg, dtype=np.uint32) if pages_of is None else np.asarray(pages_of, np.uint32)
    arena = OracleArena(npages or int(pt.max()) + 1, page, hkv, D, f16=True)
    slots = np.array([pt[i // page] * page + i % page for i in range(n)], np.uint32)
    arena.store(slots, keys.reshape(n, -1), vals.reshape(n, -1))
    return arena, pt


def test_one_key_gives_v():
    rng = np.random.default_rng(1)
    k = rng.standard_normal((1, 1, D)).astype(np.float32)
    v = rng.standard_normal((1, 1, D)).astype(np.float32)
    arena, pt = _arena_with(k, v)
    q = rng.standard_normal((1, D)).astype(np.float32)
    o = arena.attend(q, 1, [0], [0], pt)
    vb = v.reshape(-1).astype(np.float16).astype(np.float32)
    assert np.array_equal(o[0], vb)


def test_equal_scores_give_the_mean_of_v():
    rng = np.random.default_rng(2)
    n = 300
    k = rng.standard_normal((n, 1, D)).astype(np.float32)
    v = rng.standard_normal((n, 1, D)).astype(np.float32)
    arena, pt = _arena_with(k, v)
    o = arena.attend(np.zeros((1, D), np.float32), 1, [n - 1], [0], pt)
    mean = v.reshape(n, D).astype(np.float16).astype(np.float64).mean(0)
    assert np.abs(o[0] - mean).max() < 1e-5


def test_page_placement_and_wide_windows_change_nothing():
    rng = np.random.default_rng(3)
    n, hq, hkv = 777, 8, 2
    k = rng.standard_normal((n, hkv, D)).astype(np.float32)
    v = rng.standard_normal((n, hkv, D)).astype(np.float32)
    q = rng.standard_normal((1, hq * D)).astype(np.float32)
    a1, pt1 = _arena_with(k, v, hkv=hkv)
    perm = rng.permutation(200)[:len(pt1)]
    a2, pt2 = _arena_with(k, v, hkv=hkv, pages_of=perm, npages=200)
    o1 = a1.attend(q, hq, [n - 1], [0], pt1)
    o2 = a2.attend(q, hq, [n - 1], [0], pt2)
    o3 = a1.attend(q, hq, [n - 1], [0], pt1, window=n)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(o1.view(np.uint32), o3.view(np.uint32))


def test_two_pass_f32_is_close_to_f64_at_long_context():
    rng = np.random.default_rng(4)
    n, hq, hkv = 4096, 16, 4
    k = rng.standard_normal((n, hkv, D)).astype(np.float32)
    v = rng.standard_normal((n, hkv, D)).astype(np.float32)
    q = rng.standard_normal((2, hq * D)).astype(np.float32)
    arena, pt = _arena_with(k, v, hkv=hkv)
    pos = [n - 1, 1000]
    o = arena.attend(q, hq, pos, [0, 0], pt, threads=4)
    e = arena.attend_f64(q, hq, pos, [0, 0], pt)
    assert np.abs(o - e).max() < 1e-5
