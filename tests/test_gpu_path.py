"""GPU parity of the KV path against the CPU oracle (through the C ABI).

Bit-exact: appended K/V bytes, page copies. Tolerance (2e-3 abs + 1e-3 rel, f16 KV
with f32 accumulation): attention outputs vs the f32 restatement of
`LayerPass::attend` (crates/yaxus-backend-cpu/src/lib.rs:389-427) on the same f16 K/V.
"""

import contextlib

import numpy as np
import pytest

from tests.scenario import D, Scenario, close

pytestmark = pytest.mark.gpu


def _check_pages(sc, layer, pages):
    k, v = sc.kv.read_pages(layer, pages)
    for i, p in enumerate(pages):
        ok, ov = sc.orc[layer].page_bits(p)
        assert np.array_equal(k[i], ok), f"K bits differ on page {p}"
        assert np.array_equal(v[i], ov), f"V bits differ on page {p}"


def test_append_is_bit_exact(hip):
    sc = Scenario(hip, pages=64, page=16, hkv=4, pool_seed=3)
    a, b = sc.cache.new_seq(), sc.cache.new_seq()
    sc.prefill({a: 37, b: 70})
    used = sorted(set(sc.cache.seq_pages(a)) | set(sc.cache.seq_pages(b)))
    _check_pages(sc, 0, used)


def test_append_rounds_special_values(hip):
    """Round-to-nearest-even ties, subnormals, overflow and signed zeros."""
    from oracle.attn import f32_to_f16_bits

    sc = Scenario(hip, pages=4, page=16, hkv=1)
    s = sc.cache.new_seq()
    pr = sc.run_pass([(s, 16)])
    vals = np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 65519.99, 1e-8, -1e-8, 2.0 ** -24,
                     2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -14, 1.00048828125, 1.00146484375,
                     -2.5e-6, 6e-5], np.float32)
    rng = np.random.default_rng(0)
    k = rng.standard_normal((16, 1, D)).astype(np.float32) * np.float32(3e-5)
    k[:, 0, :16] = vals
    v = (rng.standard_normal((16, 1, D)) * 1e4).astype(np.float32)
    hip.append(sc.kv, 0, k, v)
    kb, vb = sc.kv.read_pages(0, [int(pr.meta.pages[0])])
    assert np.array_equal(kb[0, 0], f32_to_f16_bits(k[:, 0, :]))
    assert np.array_equal(vb[0, 0], f32_to_f16_bits(v[:, 0, :]))
    with np.errstate(over="ignore"):
        assert np.array_equal(f32_to_f16_bits(vals), vals.astype(np.float16).view(np.uint16))


def test_copy_pages_in_order(hip):
    sc = Scenario(hip, pages=8, page=16, hkv=2, layers=2)
    s = sc.cache.new_seq()
    sc.prefill({s: 5 * 16})
    from yaxus_amd import PageCopy

    # A chain: 0 -> 5, then 5 -> 6 must see the first copy's result; 1 -> 0 after 0 is read.
    copies = [PageCopy(0, 5), PageCopy(5, 6), PageCopy(1, 0)]
    hip.copy_pages(sc.kv, copies)
    for c in copies:
        for o in sc.orc:
            o.copy_page(c.src, c.dst)
    for layer in range(2):
        _check_pages(sc, layer, list(range(8)))


@contextlib.contextmanager
def option(hip, key, value):
    hip.set_option(key, value)
    try:
        yield
    finally:
        hip.set_option(key, 0)


# attn_decode_shape: 0 = the balanced one-tile kernel where it applies (waves share a
# queue of quads) and the 16-row-tile kernel for more logical rows, 1 = the 8-row-tile
# static-split kernels only.
@pytest.mark.parametrize("shape", [0, 1])
@pytest.mark.parametrize("page", [16, 32, 64, 128])
@pytest.mark.parametrize("window", [0, 100])
def test_decode_matches_oracle(hip, page, window, shape):
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=256 * 16 // page + 16, page=page, hkv=hkv, pool_seed=11)
    lens = [1, 15, 16, 17, 300, 1000, 33, 250]
    seqs = [sc.cache.new_seq() for _ in lens]
    sc.prefill(dict(zip(seqs, lens)))
    pr = sc.run_pass([(s, 1) for s in seqs])
    sc.store(pr)
    rows = len(seqs)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    with option(hip, "attn_decode_shape", shape):
        got = hip.attend(sc.kv, 0, q, hq, window=window)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    err = np.abs(got - want).max()
    assert close(got, want).all(), f"max abs err {err}"


@pytest.mark.parametrize("shape", [0, 1])
@pytest.mark.parametrize("target_waves", [1, 64, 4096])
def test_split_count_does_not_change_results(hip, target_waves, shape):
    hq, hkv = 8, 2
    sc = Scenario(hip, pages=160, page=16, hkv=hkv, pool_seed=5)
    seqs = [sc.cache.new_seq() for _ in range(3)]
    sc.prefill(dict(zip(seqs, [700, 1200, 64])))
    pr = sc.run_pass([(s, 1) for s in seqs])
    sc.store(pr)
    q = sc.draw(3 * hq * D).reshape(3, hq * D)
    with option(hip, "attn_target_waves", target_waves), option(hip, "attn_decode_shape", shape):
        got = hip.attend(sc.kv, 0, q, hq)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"


@pytest.mark.parametrize("lens", [[511], [511] * 4, [1023, 1023], [255] * 8, [40, 500, 7, 300]])
def test_tiny_passes_split_finely(hip, lens):
    """Tiny decode passes (at most two 16-key blocks per CU) take one-quad work items,
    up to 8 chunks per group: against the oracle, bit for bit from call to call, and
    within tolerance of the same pass split at the coarser default of larger passes."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=sum(lens) // 16 + 16 * len(lens), page=16, hkv=hkv, pool_seed=13)
    seqs = [sc.cache.new_seq() for _ in lens]
    sc.prefill(dict(zip(seqs, lens)))
    pr = sc.run_pass([(s, 1) for s in seqs])
    sc.store(pr)
    q = sc.draw(len(lens) * hq * D).reshape(len(lens), hq * D)
    got = hip.attend(sc.kv, 0, q, hq)
    again = hip.attend(sc.kv, 0, q, hq)
    with option(hip, "attn_target_waves", 64):  # one item per group or few chunks
        coarse = hip.attend(sc.kv, 0, q, hq)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    assert np.abs(got - coarse).max() < 2e-5
    sc.kv.destroy()


@pytest.mark.parametrize("shape", [0, 1])
@pytest.mark.parametrize("hq,hkv,k", [(16, 4, 6), (16, 4, 5), (16, 4, 7), (8, 8, 3), (16, 1, 2),
                                      (32, 1, 1), (12, 4, 4)])
def test_verify_rows_are_causal(hip, hq, hkv, k, shape):
    """Multi-row passes per sequence (speculative verify): rows see keys <= their pos.
    (16, 4, 7): 28 logical rows, one work item in the 16-row-tile kernel, two in the
    8-row one."""
    sc = Scenario(hip, pages=128, page=16, hkv=hkv, pool_seed=9)
    seqs = [sc.cache.new_seq() for _ in range(4)]
    sc.prefill(dict(zip(seqs, [40, 513, 7, 260])))
    pr = sc.run_pass([(s, k) for s in seqs])
    sc.store(pr)
    rows = len(pr.meta.pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    with option(hip, "attn_decode_shape", shape):
        got = hip.attend(sc.kv, 0, q, hq, window=0)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"


def test_attention_close_to_f64(hip):
    """The device result is closer to the f64 brute force than the tolerance by far."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=400, page=16, hkv=hkv, pool_seed=2)
    seqs = [sc.cache.new_seq() for _ in range(4)]
    sc.prefill(dict(zip(seqs, [4095, 2000, 17, 1])))
    pr = sc.run_pass([(s, 1) for s in seqs])
    sc.store(pr)
    q = sc.draw(4 * hq * D).reshape(4, hq * D)
    got = hip.attend(sc.kv, 0, q, hq)
    exact = sc.orc[0].attend_f64(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert np.abs(got - exact).max() < 2e-5


@pytest.mark.parametrize("shape", [0, 1])
@pytest.mark.parametrize("hq,hkv,k,window", [(16, 4, 1, 0), (16, 4, 5, 0), (16, 4, 6, 50),
                                             (32, 1, 2, 0), (8, 2, 3, 0)])
def test_fused_append_attention(hip, hq, hkv, k, window, shape):
    """One launch stores the rows' K/V and attends (the append falls back to its own
    kernel when a sequence's rows do not fit one work item: hq=32, hkv=1, k=2)."""
    sc = Scenario(hip, pages=200, page=16, hkv=hkv, pool_seed=4)
    seqs = [sc.cache.new_seq() for _ in range(5)]
    sc.prefill(dict(zip(seqs, [0 + 1, 64, 300, 1023, 15])))
    pr = sc.run_pass([(s, k) for s in seqs])
    rows = len(pr.meta.pos)
    kk = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    vv = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    with option(hip, "attn_decode_shape", shape):
        got = hip.attend_append(sc.kv, 0, kk, vv, q, hq, window=window)
    sc.orc[0].store(pr.meta.kv_slot, kk.reshape(rows, -1), vv.reshape(rows, -1))
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    used = sorted(set(int(p) for s in seqs for p in sc.cache.seq_pages(s)))
    _check_pages(sc, 0, used)


@pytest.mark.parametrize("shape", [0, 1])
def test_attention_is_deterministic(hip, shape):
    """Chunks are merged in chunk order, and quads of blocks in quad order whichever
    wave ran them (or each wave's blocks are fixed): two runs give the same bits."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=800, page=16, hkv=hkv, pool_seed=8)
    seqs = [sc.cache.new_seq() for _ in range(8)]
    sc.prefill(dict(zip(seqs, [4000, 3000, 2047, 100, 1, 555, 1024, 700])))
    pr = sc.run_pass([(s, 1) for s in seqs])
    sc.store(pr)
    q = sc.draw(8 * hq * D).reshape(8, hq * D)
    with option(hip, "attn_decode_shape", shape):
        a = hip.attend(sc.kv, 0, q, hq)
        b = hip.attend(sc.kv, 0, q, hq)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("shape", [0, 1, 2])
@pytest.mark.parametrize("hq,hkv,k", [(4, 4, 1), (8, 2, 1), (16, 4, 1), (16, 2, 1), (16, 4, 3)])
def test_merge_of_many_chunks(hip, hq, hkv, k, shape):
    """Long groups cut into ~100 chunks: the last chunk's workgroup merges them in
    contiguous ranges over up to 16 thread groups (fewer with more logical rows) and
    adds the ranges in order. shape 2 forces the 16-row-tile kernel on one-tile passes."""
    sc = Scenario(hip, pages=12000 // 16 * 2 + 16, page=16, hkv=hkv, pool_seed=21)
    seqs = [sc.cache.new_seq() for _ in range(2)]
    sc.prefill(dict(zip(seqs, [12000, 5000])))
    pr = sc.run_pass([(s, k) for s in seqs])
    sc.store(pr)
    rows = len(pr.meta.pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    with option(hip, "attn_decode_shape", shape), option(hip, "attn_target_waves", 4096):
        a = hip.attend(sc.kv, 0, q, hq)
        b = hip.attend(sc.kv, 0, q, hq)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(a, want).all(), f"max abs err {np.abs(a - want).max()}"


@pytest.mark.parametrize("shape", [0, 1])
def test_verify_attention_is_deterministic(hip, shape):
    """Multi-tile work items (5 rows x 4 q heads): two runs give the same bits, and
    another split of the groups' blocks into chunks stays within the tolerance."""
    hq, hkv = 16, 4
    sc = Scenario(hip, pages=800, page=16, hkv=hkv, pool_seed=18)
    seqs = [sc.cache.new_seq() for _ in range(6)]
    sc.prefill(dict(zip(seqs, [4000, 3000, 2047, 100, 1, 555])))
    pr = sc.run_pass([(s, 5) for s in seqs])
    sc.store(pr)
    rows = len(pr.meta.pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    with option(hip, "attn_decode_shape", shape):
        a = hip.attend(sc.kv, 0, q, hq)
        b = hip.attend(sc.kv, 0, q, hq)
        with option(hip, "attn_target_waves", 4096):
            c = hip.attend(sc.kv, 0, q, hq)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(a, want).all() and close(c, want).all()


@pytest.mark.parametrize("hq,hkv,page,window,chunk", [
    (16, 4, 16, 0, 256), (16, 4, 16, 100, 64), (8, 8, 16, 0, 40), (32, 2, 128, 0, 96),
    (16, 4, 128, 300, 33), (16, 4, 32, 0, 70), (8, 2, 64, 50, 129)])
def test_prefill_tiles_match_oracle(hip, hq, hkv, page, window, chunk):
    """Chunked prefill (many rows per sequence): the MFMA tile kernel over LDS-staged
    K/V, causal within the chunk and full (or windowed) over the earlier context."""
    sc = Scenario(hip, pages=420 * 16 // page + 12, page=page, hkv=hkv, pool_seed=12)
    prior = [8, 0, 1000, 517]
    seqs = [sc.cache.new_seq() for _ in prior]
    sc.prefill({s: n for s, n in zip(seqs, prior) if n})
    pr = sc.run_pass([(s, chunk) for s in seqs])
    rows = len(pr.meta.pos)
    kk = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    vv = sc.draw(rows * hkv * D).reshape(rows, hkv, D)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    before = hip.stat("prefill_plans")
    hip.set_option("prefill_min_rows", 1)  # the tile kernel whatever the automatic choice
    try:
        got = hip.attend_append(sc.kv, 0, kk, vv, q, hq, window=window)
    finally:
        hip.set_option("prefill_min_rows", 0)
    assert hip.stat("prefill_plans") == before + 1
    sc.orc[0].store(pr.meta.kv_slot, kk.reshape(rows, -1), vv.reshape(rows, -1))
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    err = np.abs(got - want).max()
    assert close(got, want).all(), f"max abs err {err}"
    assert err < 2e-5, f"max abs err {err}"


@pytest.mark.parametrize("hq,hkv,page,window,prior,chunk,f32", [
    (16, 4, 16, 0, 3000, 64, 0), (16, 4, 16, 2000, 3000, 64, 0),
    (8, 2, 32, 0, 5000, 33, 0), (32, 2, 16, 0, 2500, 40, 0),
    (16, 4, 64, 0, 4100, 256, 0), (16, 4, 16, 0, 4000, 64, 8),
    (8, 2, 32, 1500, 5000, 130, 8), (16, 4, 16, 0, 4000, 64, 4),
    (8, 2, 32, 1500, 5000, 130, 4)])
def test_prefill_split_along_keys(hip, hq, hkv, page, window, prior, chunk, f32):
    """One long sequence's chunk: too few tiles to fill the GPU, so each tile's keys are
    split over several work items whose partial softmaxes the tile's last chunk merges.
    Against the oracle (to 2e-5), against the same pass with the split off, and bit for
    bit from call to call (the merge runs in chunk order). A second, short sequence in
    the same pass keeps its tiles whole. Both arenas (binary16, and f32 with its own
    prefill kernel, in tiles of 128 and of 64 logical rows: f32 = its waves)."""
    sc = Scenario(hip, pages=(prior + chunk) // page + 64, page=page, hkv=hkv, pool_seed=7, f32=bool(f32))
    a, b = sc.cache.new_seq(), sc.cache.new_seq()
    sc.prefill({a: prior, b: 40})
    pr = sc.run_pass([(a, chunk), (b, 20)])
    sc.store(pr)
    rows = len(pr.meta.pos)
    q = sc.draw(rows * hq * D).reshape(rows, hq * D)
    want = sc.orc[0].attend(q, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
    hip.set_option("prefill_min_rows", 1)  # the prefill kernel (few tiles: decode by default)
    hip.set_option("prefill_f32_waves", f32)
    try:
        split0 = hip.stat("prefill_split_tiles")
        got = hip.attend(sc.kv, 0, q, hq, window=window)
        assert hip.stat("prefill_split_tiles") > split0  # the long sequence's tiles were split
        again = hip.attend(sc.kv, 0, q, hq, window=window)
        hip.set_option("prefill_split", 0)
        try:
            whole = hip.attend(sc.kv, 0, q, hq, window=window)
        finally:
            hip.set_option("prefill_split", 1)
    finally:
        hip.set_option("prefill_min_rows", 0)
        hip.set_option("prefill_f32_waves", 0)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    for x in (got, whole):
        err = np.abs(x - want).max()
        assert close(x, want).all() and err < 2e-5, f"max abs err {err}"
    assert np.abs(got - whole).max() < 2e-5
    sc.kv.destroy()


def test_prefill_split_through_backend_attention(hip):
    """Backend::attention in full (write_rows' key heads, then the prefill kernel, which
    normalises and rotates its q heads itself) on a long sequence's chunk whose tiles
    are split along keys: against write_rows + attention in the oracle."""
    from yaxus_amd.rope import inv_freq, rope_table

    hq, hkv = 16, 4
    sc = Scenario(hip, pages=3200 // 16 + 16, page=16, hkv=hkv, pool_seed=9)
    s = sc.cache.new_seq()
    sc.prefill({s: 3000})
    pr = sc.run_pass([(s, 64)])
    rows = len(pr.meta.pos)
    qkv = sc.draw(rows * (hq + 2 * hkv) * D).reshape(rows, -1)
    qn, kn = sc.draw(D) * 0.1, sc.draw(D) * 0.1
    f = inv_freq(D, 10000.0)
    hip.set_option("prefill_min_rows", 1)  # the prefill kernel (few tiles: decode by default)
    try:
        split0 = hip.stat("prefill_split_tiles")
        got = hip.attention(sc.kv, 0, qkv, qn, kn, rope_table(f, 1.0, 4096), 1e-6, hq)
        assert hip.stat("prefill_split_tiles") > split0
    finally:
        hip.set_option("prefill_min_rows", 0)
    qo = sc.orc[0].write_rows(qkv, hq, qn, kn, 1e-6, f, 1.0, pr.meta.pos, pr.meta.kv_slot)
    want = sc.orc[0].attend(qo, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    err = np.abs(got - want).max()
    assert close(got, want).all() and err < 2e-5, f"max abs err {err}"
    sc.kv.destroy()


@pytest.mark.parametrize("hq,hkv,page,lens,k", [
    (16, 4, 16, [1, 300, 17, 64], 1), (8, 8, 16, [5, 40], 33), (32, 2, 128, [200, 1], 3),
    (16, 1, 16, [0, 1000], 2)])
def test_qk_rope_append_matches_write_rows(hip, hq, hkv, page, lens, k):
    """write_rows on the device (RMSNorm + RoPE of q and k, K/V store) gives the CPU
    backend's bits: q as f32, K and V as their binary16 roundings (orc_write_rows)."""
    from oracle.attn import cos_sin_table
    from yaxus_amd.rope import inv_freq, rope_table

    sc = Scenario(hip, pages=200 if page == 16 else 40, page=page, hkv=hkv, pool_seed=6)
    seqs = [sc.cache.new_seq() for _ in lens]
    sc.prefill({s: n for s, n in zip(seqs, lens) if n > 0})
    pr = sc.run_pass([(s, k) for s in seqs])
    rows = len(pr.meta.pos)
    qkv = (sc.draw(rows * (hq + 2 * hkv) * D) * 3.0).reshape(rows, -1)
    qn = sc.draw(D) * 0.1
    kn = sc.draw(D) * 0.1
    f = inv_freq(D, 10000.0)
    conc = 1.2079441
    table = rope_table(f, conc, 2048)
    assert np.array_equal(table.view(np.uint32), cos_sin_table(f, conc, 2048).view(np.uint32))
    q = hip.qk_rope_append(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
    want = sc.orc[0].write_rows(qkv, hq, qn, kn, 1e-6, f, conc, pr.meta.pos, pr.meta.kv_slot)
    assert np.array_equal(q.view(np.uint32), want.view(np.uint32)), \
        f"{(q.view(np.uint32) != want.view(np.uint32)).sum()} q values differ, max {np.abs(q - want).max()}"
    written = sorted(set(int(s) // page for s in pr.meta.kv_slot))
    _check_pages(sc, 0, written)


def test_qk_rope_append_rejects_positions_past_the_table(hip):
    from yaxus_amd._lib import YxError
    from yaxus_amd.rope import inv_freq, rope_table

    sc = Scenario(hip, pages=40, page=16, hkv=2)
    s = sc.cache.new_seq()
    sc.prefill({s: 100})
    sc.run_pass([(s, 1)])
    qkv = np.zeros((1, (8 + 4) * D), np.float32)
    with pytest.raises(YxError, match="RoPE table"):
        hip.qk_rope_append(sc.kv, 0, qkv, np.zeros(D), np.zeros(D),
                           rope_table(inv_freq(D, 10000.0), 1.0, 64), 1e-6, 8)


@pytest.mark.parametrize("window", [None, 16])
def test_model_attention_two_passes_across_pages(hip, window):
    """backend-cpu lib.rs:676-714 at head_dim 128 on the device: two sequences on the
    non-adjacent pages [3, 1] and [0], lengths 140 and 9, written in two passes that
    cross a page boundary (PAGE = 128), through Backend::attention in full (write_rows
    then attend), against the oracle's write_rows + attend on the same f16 arena."""
    from types import SimpleNamespace

    from oracle.attn import OracleArena
    from tests.test_attn_oracle import _values
    from yaxus_amd.rope import rope_table

    hq, hkv, P, eps = 4, 2, 128, 1e-6
    f = np.array([1.0 / 10000.0 ** (i / 64) for i in range(64)], np.float32)
    conc = 1.1
    table = rope_table(f, conc, 256)
    cols = (hq + 2 * hkv) * D
    pages = [[3, 1], [0]]
    lens = [140, 9]
    qkv = [[_values(cols, s * 1000 + p) for p in range(n)] for s, n in enumerate(lens)]
    qn = _values(D, 7) * np.float32(0.5)
    kn = _values(D, 8) * np.float32(0.5)
    kv = hip.new_kv(1, 4, P, hkv)
    orc = OracleArena(4, P, hkv, D, f16=True)
    first = [(0, p) for p in range(100)] + [(1, p) for p in range(4)]
    second = [(0, p) for p in range(100, 140)] + [(1, p) for p in range(4, 9)]
    for rows in (first, second):
        meta_pages, off = [], {}
        for sq, _ in rows:
            if sq not in off:
                off[sq] = len(meta_pages)
                meta_pages += pages[sq]
        meta = SimpleNamespace(
            pos=np.array([p for _, p in rows], np.uint32),
            kv_slot=np.array([pages[s][p // P] * P + p % P for s, p in rows], np.uint32),
            pt_off=np.array([off[s] for s, _ in rows], np.uint32),
            pages=np.array(meta_pages, np.uint32))
        x = np.stack([qkv[s][p] for s, p in rows])
        hip.begin_pass(meta)
        got = hip.attention(kv, 0, x, qn, kn, table, eps, hq, window=window)
        q = orc.write_rows(x, hq, qn, kn, eps, f, conc, meta.pos, meta.kv_slot)
        want = orc.attend(q, hq, meta.pos, meta.pt_off, meta.pages, window=window or 0)
        assert close(got, want).all(), f"max abs err {np.abs(got - want).max()}"
    k, v = kv.read_pages(0, [0, 1, 3])
    for i, p in enumerate([0, 1, 3]):
        ok, ov = orc.page_bits(p)
        assert np.array_equal(k[i], ok) and np.array_equal(v[i], ov)
    kv.destroy()


@pytest.mark.parametrize("hq,hkv,lens,k,min_rows", [
    (16, 4, [1, 300, 17, 1000, 64], 1, 0), (8, 2, [40, 513], 1, 0), (16, 4, [40, 513, 7], 5, 0),
    (32, 2, [100, 2000], 1, 0), (16, 4, [40, 513, 7], 40, 0), (8, 8, [0, 130], 70, 0),
    (16, 4, [40, 513, 7], 40, 32), (8, 8, [0, 130], 70, 32),
    (16, 4, [4095], 1, 0), (16, 4, [40, 513, 7], 4, 0)])
def test_attention_in_one_launch_equals_two(hip, request, hq, hkv, lens, k, min_rows):
    """Backend::attention in full gives the same bits (attention output and stored K/V)
    as write_rows then attention as separate calls, and both match the oracle: decode
    passes in one launch (the decode kernel runs write_rows itself: the queue kernel, or
    the 16-row-tile kernel for [4095], whose 8-quad work items split evenly over its
    waves, and for k = 4, 16 logical rows), verify passes of more rows (k = 5) as
    write_rows then attention, prefill passes (k >= 32 with min_rows 32; automatically
    these few tiles are decode items) as the key heads' write_rows then the prefill
    kernel, which normalises and rotates its q heads itself."""
    from yaxus_amd.rope import inv_freq, rope_table

    f = inv_freq(D, 10000.0)
    table = rope_table(f, 1.0, 4096)
    outs, scs = [], []
    hip.set_option("prefill_min_rows", min_rows)
    request.addfinalizer(lambda: hip.set_option("prefill_min_rows", 0))
    for one_launch in (True, False):
        sc = Scenario(hip, pages=400, page=16, hkv=hkv, pool_seed=21)
        seqs = [sc.cache.new_seq() for _ in lens]
        sc.prefill({s: n for s, n in zip(seqs, lens) if n})
        pr = sc.run_pass([(s, k) for s in seqs])
        rows = len(pr.meta.pos)
        qkv = sc.draw(rows * (hq + 2 * hkv) * D).reshape(rows, -1)
        qn, kn = sc.draw(D) * 0.1, sc.draw(D) * 0.1
        if one_launch:
            got = hip.attention(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
        else:
            q = hip.qk_rope_append(sc.kv, 0, qkv, qn, kn, table, 1e-6, hq)
            got = hip.attend(sc.kv, 0, q, hq)
        outs.append(got)
        scs.append((sc, pr))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    (sa, pr), (sb, _) = scs
    written = sorted(set(int(s) // 16 for s in pr.meta.kv_slot))
    ka, va = sa.kv.read_pages(0, written)
    kb, vb = sb.kv.read_pages(0, written)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    # The oracle on a third, identical scenario (same seeds, so the same inputs).
    rows = len(pr.meta.pos)
    sc = Scenario(hip, pages=400, page=16, hkv=hkv, pool_seed=21)
    seqs = [sc.cache.new_seq() for _ in lens]
    sc.prefill({s: n for s, n in zip(seqs, lens) if n})
    pr = sc.run_pass([(s, k) for s in seqs])
    qkv = sc.draw(rows * (hq + 2 * hkv) * D).reshape(rows, -1)
    qn, kn = sc.draw(D) * 0.1, sc.draw(D) * 0.1
    qo = sc.orc[0].write_rows(qkv, hq, qn, kn, 1e-6, f, 1.0, pr.meta.pos, pr.meta.kv_slot)
    want = sc.orc[0].attend(qo, hq, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    assert close(outs[0], want).all(), f"max abs err {np.abs(outs[0] - want).max()}"


def test_dev_checksum_is_the_xor_of_the_words(hip):
    """yx_dev_checksum = XOR of every 8-byte word (numpy), including a size that leaves
    threads without work and the empty buffer."""
    rng = np.random.default_rng(11)
    for n in (16, 4096 + 48, 1 << 22):
        a = rng.integers(0, 2**63, size=n // 8, dtype=np.uint64)
        t = hip.tensor((n,), np.uint8).upload(a.view(np.uint8))
        try:
            assert hip.checksum(t.ptr, n) == int(np.bitwise_xor.reduce(a))
        finally:
            t.free()
    assert hip.checksum(None, 0) == 0
