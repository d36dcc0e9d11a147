"""The f32 arena (`yx_kv_create` with YX_DTYPE_F32): K/V kept in the reference's own
precision (CpuBackend::new_kv, crates/yaxus-backend-cpu/src/lib.rs:464-470, holds f32),
attended by the f32-MFMA decode kernel and, for passes with many rows per sequence, the
f32-MFMA prefill kernel (exact f32 products, f32 accumulation, both). Stores are
bit-exact; attention is within the path's tolerance of the oracle's f32 arena and within
1e-5 of the f64 brute force (the reference's own paged-vs-dense bound,
crates/yaxus-backend-cpu/src/lib.rs:709)."""

import contextlib

import numpy as np
import pytest

from tests.scenario import D, Scenario, close

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _check_pages(sc, layer, pages):
    k, v = sc.kv.read_pages(layer, pages)
    for i, p in enumerate(pages):
        ok, ov = sc.orc[layer].page_bits(int(p))
        assert np.array_equal(k[i], _bits(ok)) and np.array_equal(v[i], _bits(ov)), f"page {p}"


@pytest.mark.parametrize("page", [16, 64])
def test_f32_append_is_exact(hip, page):
    sc = Scenario(hip, pages=64 * 16 // page + 8, page=page, hkv=4, pool_seed=3, f32=True)
    seqs = [sc.cache.new_seq() for _ in range(3)]
    sc.prefill(dict(zip(seqs, [1, 37, 300])))
    used = sorted({int(p) for s in seqs for p in sc.cache.seq_pages(s)})
    _check_pages(sc, 0, used)
    sc.kv.destroy()


@pytest.mark.parametrize("hq,hkv", [(16, 4), (8, 8), (16, 1), (12, 4)])
@pytest.mark.parametrize("page,window", [(16, 0), (32, 100), (128, 0)])
@pytest.mark.parametrize("k", [1, 5])
def test_f32_decode_and_verify_match_oracle(hip, hq, hkv, page, window, k):
    sc = Scenario(hip, pages=3000 * 2 // page + 40, page=page, hkv=hkv, pool_seed=7, f32=True)
    lens = [1, 16, 17, 300, 2999, 64]
    seqs = [sc.cache.new_seq() for _ in lens]
    sc.prefill(dict(zip(seqs, lens)))
    pr = sc.run_pass([(s, k) for s in seqs])
    rows = len(pr.meta.pos)
    kk = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    vv = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    got = hip.attend_append(sc.kv, 0, kk, vv, q, hq, window=window)
    sc.orc[0].store(pr.meta.kv_slot, kk.reshape(rows, -1), vv.reshape(rows, -1))
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    exact = sc.orc[0].attend_f64(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    assert np.abs(got - exact).max() < 1e-5
    used = sorted({int(p) for s in seqs for p in sc.cache.seq_pages(s)})
    _check_pages(sc, 0, used)
    sc.kv.destroy()


@pytest.fixture(autouse=True, params=[8, 4], ids=["tiles128", "tiles64"])
def _prefill_from_32_rows(hip, request):
    """The prefill kernel for every pass with 32 or more rows of one sequence (the
    automatic choice would attend these small passes as decode items), with tiles of
    128 logical rows (8 waves) and of 64 (4 waves, two workgroups per CU)."""
    hip.set_option("prefill_min_rows", 32)
    hip.set_option("prefill_f32_waves", request.param)
    yield
    hip.set_option("prefill_min_rows", 0)
    hip.set_option("prefill_f32_waves", 0)


@contextlib.contextmanager
def _option(hip, key, value, default):
    hip.set_option(key, value)
    try:
        yield
    finally:
        hip.set_option(key, default)


def test_f32_prefill_rows_and_determinism(hip):
    """Many rows per sequence (a prefill chunk) take the f32 prefill kernel; two runs give
    the same bits."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=200, page=16, hkv=hkv, pool_seed=5, f32=True)
    seqs = [sc.cache.new_seq() for _ in range(3)]
    sc.prefill(dict(zip(seqs, [0 + 8, 700, 33])))
    pr = sc.run_pass([(s, 48) for s in seqs])
    sc.store(pr)
    rows = len(pr.meta.pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    a = hip.attend(sc.kv, 0, q, hq)
    b = hip.attend(sc.kv, 0, q, hq)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(a, want).all(), f"max abs err {np.abs(a - want).max()}"
    sc.kv.destroy()


def test_f32_write_rows_and_attention(hip):
    """Backend::attention on an f32 arena: write_rows stores the key heads as computed
    (the oracle's f32 bits) and the raw value heads; q is bit-exact; the attention
    matches the oracle."""
    from yaxus_amd.rope import inv_freq, rope_table

    hq, hkv = 16, 4
    f = inv_freq(D, 10000.0)
    table = rope_table(f, 1.0, 4096)
    sc = Scenario(hip, pages=200, page=16, hkv=hkv, pool_seed=9, f32=True)
    seqs = [sc.cache.new_seq() for _ in range(4)]
    sc.prefill(dict(zip(seqs, [5, 300, 1000, 40])))
    pr = sc.run_pass([(s, 1) for s in seqs])
    rows = len(pr.meta.pos)
    qkv = sc.draw(rows * (hq + 2 * hkv) * D).reshape(rows, -1)
    qn, kn = sc.draw(D) * 0.1, sc.draw(D) * 0.1
    q = hip.qk_rope_append(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
    qo = sc.orc[0].write_rows(qkv, hq, qn, kn, 1e-6, f, 1.0, pr.meta.pos, pr.meta.kv_slot)
    assert np.array_equal(q.view(np.uint32), qo.view(np.uint32))
    _check_pages(sc, 0, sorted({int(s) // 16 for s in pr.meta.kv_slot}))
    got = hip.attention(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
    want = sc.orc[0].attend(qo, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    sc.kv.destroy()


def test_f32_copy_pages(hip):
    """Copy-on-write of a shared tail page in the f32 arena: the copy is bit-exact."""
    sc = Scenario(hip, pages=64, page=16, hkv=2, pool_seed=4, f32=True)
    base = sc.cache.new_seq()
    sc.prefill({base: 40})
    copies = []
    fork = sc.cache.fork(base, 40, copies)
    assert copies, "a partial tail page is copied"
    sc.hip.copy_pages(sc.kv, copies)
    for c in copies:
        sc.orc[0].copy_page(c.src, c.dst)
    _check_pages(sc, 0, sorted({c.dst for c in copies} | {c.src for c in copies}))
    assert fork is not None
    sc.kv.destroy()


@pytest.mark.parametrize("hq,hkv,page,window,chunk", [
    (16, 4, 16, 0, 256), (16, 4, 16, 100, 64), (8, 8, 16, 0, 40), (32, 2, 128, 0, 96),
    (16, 4, 128, 300, 33), (16, 4, 32, 0, 70), (8, 2, 64, 50, 129), (12, 4, 16, 0, 50)])
def test_f32_prefill_tiles_match_oracle(hip, hq, hkv, page, window, chunk):
    """Chunked prefill over the f32 arena (the prefill kernel's exact f32 products): the
    oracle's f32 arena within tolerance, the f64 brute force within 1e-5, and the f32
    decode kernel (the same pass with prefill tiles switched off) within 1e-5."""
    sc = Scenario(hip, pages=420 * 16 // page + 12, page=page, hkv=hkv, pool_seed=12, f32=True)
    prior = [8, 0, 1000, 517]
    seqs = [sc.cache.new_seq() for _ in prior]
    sc.prefill({s: n for s, n in zip(seqs, prior) if n})
    pr = sc.run_pass([(s, chunk) for s in seqs])
    rows = len(pr.meta.pos)
    kk = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    vv = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    got = hip.attend_append(sc.kv, 0, kk, vv, q, hq, window=window)
    sc.orc[0].store(pr.meta.kv_slot, kk.reshape(rows, -1), vv.reshape(rows, -1))
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    exact = sc.orc[0].attend_f64(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    assert np.abs(got - exact).max() < 1e-5
    with _option(hip, "prefill_min_rows", 1 << 20, 32):
        split = hip.attend(sc.kv, 0, q, hq, window=window)
    assert np.abs(got - split).max() < 1e-5
    sc.kv.destroy()


def test_f32_prefill_values_beyond_binary16_range(hip):
    """K and V far outside binary16's range (|V| up to ~4e6, scores in the hundreds):
    the f32 prefill kernel rounds no operand to a narrower type, so the result follows
    the f64 brute force to f32 precision."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=200, page=16, hkv=hkv, pool_seed=21, f32=True)
    seqs = [sc.cache.new_seq() for _ in range(3)]
    sc.prefill(dict(zip(seqs, [100, 0, 600])))
    pr = sc.run_pass([(s, 64) for s in seqs])
    rows = len(pr.meta.pos)
    kk = (sc.draw(rows * hkv * D) * 30.0).reshape(rows, hkv, D)
    vv = (sc.draw(rows * hkv * D) * 1.0e6).reshape(rows, hkv, D)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    got = hip.attend_append(sc.kv, 0, kk, vv, q, hq)
    sc.orc[0].store(pr.meta.kv_slot, kk.reshape(rows, -1), vv.reshape(rows, -1))
    assert np.isfinite(got).all()
    exact = sc.orc[0].attend_f64(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    scale = np.abs(vv).max()
    assert scale > 65504.0 * 10
    assert np.abs(got - exact).max() < 1e-5 * scale
    sc.kv.destroy()


def test_f32_backend_attention_prefill_chunk(hip):
    """Backend::attention over an f32 arena for a 48-row chunk per sequence: write_rows,
    then the prefill kernel on its q; the oracle's write_rows plus attend agree."""
    from yaxus_amd.rope import inv_freq, rope_table

    hq, hkv = 16, 4
    f = inv_freq(D, 10000.0)
    table = rope_table(f, 1.0, 4096)
    sc = Scenario(hip, pages=200, page=16, hkv=hkv, pool_seed=13, f32=True)
    seqs = [sc.cache.new_seq() for _ in range(3)]
    sc.prefill(dict(zip(seqs, [5, 300, 0])))
    pr = sc.run_pass([(s, 48) for s in seqs])
    rows = len(pr.meta.pos)
    qkv = sc.draw(rows * (hq + 2 * hkv) * D).reshape(rows, -1)
    qn, kn = sc.draw(D) * 0.1, sc.draw(D) * 0.1
    got = hip.attention(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
    qo = sc.orc[0].write_rows(qkv, hq, qn, kn, 1e-6, f, 1.0, pr.meta.pos, pr.meta.kv_slot)
    want = sc.orc[0].attend(qo, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    _check_pages(sc, 0, sorted({int(s) // 16 for s in pr.meta.kv_slot}))
    sc.kv.destroy()
