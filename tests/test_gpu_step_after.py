"""The step after attention on the GPU against the CPU backend's restatement
(oracle/attn_oracle.c): Backend::matmul with a bf16 weight (the output projection;
crates/yaxus-backend-cpu/src/lib.rs:234-248, 314-345) within f32 accumulation error of
the oracle, and argmax_rows (lib.rs:432-440) bit for bit, over the decode shapes and
edge cases (partial tiles, ties, NaN, infinities, signed zeros, one column)."""

import numpy as np
import pytest

from oracle.attn import argmax_rows, matmul_bf16, normal

pytestmark = pytest.mark.gpu


def _bf16_bits(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("t,k,n", [(1, 2048, 2048), (16, 2048, 2048), (5, 72, 40), (17, 256, 33),
                                   (40, 2048, 256), (16, 8, 16), (3, 4096, 1000)])
def test_matmul_bf16_matches_the_cpu_backend(hip, t, k, n):
    x = normal(t * k, 31, t * 7 + n).reshape(t, k)
    w = _bf16_bits(normal(n * k, 32, k + n).reshape(n, k))
    dx = hip.tensor(x.shape).upload(x)
    dw = hip.tensor(w.shape, np.uint16).upload(w)
    try:
        got = hip.matmul_bf16(dx, dw).numpy()
    finally:
        dx.free()
        dw.free()
    want = matmul_bf16(x, w)
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    # Exact products, f32 sums in another order: within 2 k ulp-weighted magnitudes.
    bound = 2 * k * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(wf).astype(np.float64).T)
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound), np.abs(got - want).max()


def test_matmul_bf16_at_the_ends_of_the_f32_range(hip):
    """x near FLT_MAX (a rounded-up bf16 part would be inf), tiny x (down to 2^-110, the
    low parts near bf16's subnormals) and infinite x (the CPU gives +-inf, not NaN), in
    the same rows as ordinary values: within the same bound as above of the oracle, and
    the same infinities."""
    t, k, n = 4, 256, 48
    x = normal(t * k, 41, 0).reshape(t, k)
    x[0, :] *= np.float32(3.0e38) / np.abs(x[0, :]).max()    # |x| up to 3e38
    x[0, ::2] = np.float32(3.4e38)                            # above bf16's largest (3.39e38)
    x[1, :] *= np.float32(2.0 ** -100)
    x[1, 5] = np.float32(2.0 ** -110) * np.float32(1.7)
    x[2, 7] = np.inf
    w = _bf16_bits(normal(n * k, 42, 0).reshape(n, k) * np.float32(2.0 ** -10))
    w[:, 7] = _bf16_bits(np.float32(0.5))                     # row 2: +inf in every output
    dx = hip.tensor(x.shape).upload(x)
    dw = hip.tensor(w.shape, np.uint16).upload(w)
    try:
        got = hip.matmul_bf16(dx, dw).numpy()
    finally:
        dx.free()
        dw.free()
    with np.errstate(over="ignore", invalid="ignore"):
        want = matmul_bf16(x, w)
    assert np.isfinite(got[[0, 1, 3]]).all()
    assert np.array_equal(got[2], want[2]) and np.isposinf(got[2]).all()
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    fin = [0, 1, 3]
    bound = 2 * k * 2.0 ** -24 * (np.abs(x[fin]).astype(np.float64) @ np.abs(wf).astype(np.float64).T)
    bound += k * 2.0 ** -149  # the subnormal floor of the f32 sums
    assert np.all(np.abs(got[fin].astype(np.float64) - want[fin]) <= bound)


def test_argmax_rows_matches_the_cpu_backend(hip):
    rng = np.random.default_rng(9)
    cases = [rng.standard_normal((16, 151936), dtype=np.float32),
             rng.standard_normal((1, 151936), dtype=np.float32),
             rng.standard_normal((3, 1), dtype=np.float32),
             rng.standard_normal((20, 4097), dtype=np.float32)]
    a = cases[0]
    a[0, [5, 150000]] = 99.0                # a tie across slices: the first
    a[1, :] = np.nan                        # all NaN: 0
    a[2, :] = -np.inf                       # all -inf: 0
    a[3, 1000] = np.inf
    a[4, :] = np.nan
    a[4, 77777] = -3.0                      # one number among NaN
    a[5, :] = -0.0
    a[5, 100000] = 0.0                      # equal zeros: the first
    a[6, ::2] = np.nan                      # NaN interleaved
    for logits in cases:
        d = hip.tensor(logits.shape).upload(logits)
        try:
            got = hip.argmax_rows(d)
            np.testing.assert_array_equal(got.numpy(), argmax_rows(logits))
            got.free()
            # Again (the arrival counters are back at zero).
            got = hip.argmax_rows(d)
            np.testing.assert_array_equal(got.numpy(), argmax_rows(logits))
            got.free()
        finally:
            d.free()


def test_matmul_rows_do_not_depend_on_the_pass(hip):
    """Reference crates/yaxus-backend-gpu/tests/kernels.rs:250-321 (rows alone, and as rows
    of passes of 3 and 7, against the 16-row pass): a row's output has the same bits
    whatever other rows share its pass, for passes of up to 16 rows (one row tile: the
    split of k over workgroups depends only on the tile count), so batching decode rows
    cannot change a sequence's logits."""
    k, n = 1536, 200
    x = normal(16 * k, 31, 5).reshape(16, k)
    w = _bf16_bits(normal(n * k, 32, 6).reshape(n, k))
    dw = hip.tensor(w.shape, np.uint16).upload(w)

    def run(rows):
        dx = hip.tensor(rows.shape).upload(np.ascontiguousarray(rows))
        try:
            return hip.matmul_bf16(dx, dw).numpy()
        finally:
            dx.free()

    try:
        full = run(x)
        for start, t in [(0, 1), (5, 1), (15, 1), (2, 3), (8, 7)]:
            part = run(x[start:start + t])
            assert np.array_equal(part.view(np.uint32), full[start:start + t].view(np.uint32)), (start, t)
    finally:
        dw.free()


@pytest.mark.parametrize("rows", [1, 64, 65, 300, 512, 1100])
def test_argmax_handles_a_whole_pass(hip, rows):
    """Reference kernels.rs:322-343: a planted maximum per row over passes of up to 1100
    rows; a row of only -inf or only NaN gives index 0."""
    cols = 1000
    x = np.clip(normal(rows * cols, rows, 0), -4.0, 4.0).reshape(rows, cols)  # below the planted 5
    want = np.array([(r * 37) % cols for r in range(rows)], np.uint32)
    x[np.arange(rows), want] = 5.0
    if rows >= 2:
        x[0, :] = -np.inf
        x[1, :] = np.nan
        want[0] = want[1] = 0
    d = hip.tensor(x.shape).upload(x)
    try:
        got = hip.argmax_rows(d)
        np.testing.assert_array_equal(got.numpy(), want)
        np.testing.assert_array_equal(got.numpy(), argmax_rows(x))
        got.free()
    finally:
        d.free()


@pytest.mark.parametrize("slices", [1, 3, 19, 152, 1024])
def test_argmax_result_does_not_depend_on_the_slices(hip, slices):
    """The option argmax_slices (workgroups per row): every count gives the CPU's pick,
    ties across slices included; then back to the automatic count."""
    rng = np.random.default_rng(slices)
    logits = rng.standard_normal((16, 151936), dtype=np.float32)
    logits[0, [3, 151000]] = 50.0
    logits[1, :] = np.nan
    logits[2, 100000:] = 7.0
    d = hip.tensor(logits.shape).upload(logits)
    hip.set_option("argmax_slices", slices)
    try:
        for _ in range(2):  # the counters are back at zero for the next call
            got = hip.argmax_rows(d)
            np.testing.assert_array_equal(got.numpy(), argmax_rows(logits))
            got.free()
    finally:
        hip.set_option("argmax_slices", 0)
        d.free()


@pytest.mark.parametrize("ks", [1, 2, 5, 16, 64])
def test_matmul_k_split_stays_within_the_bound(hip, ks):
    """The option matmul_k_split (workgroups per output tile along k): each split is
    within the f32 accumulation bound of the oracle and repeats its own bits."""
    t, k, n = 16, 2048, 200
    x = normal(t * k, 41, ks).reshape(t, k)
    w = _bf16_bits(normal(n * k, 42, ks).reshape(n, k))
    dx = hip.tensor(x.shape).upload(x)
    dw = hip.tensor(w.shape, np.uint16).upload(w)
    hip.set_option("matmul_k_split", ks)
    try:
        a = hip.matmul_bf16(dx, dw).numpy()
        b = hip.matmul_bf16(dx, dw).numpy()
    finally:
        hip.set_option("matmul_k_split", 0)
        dx.free()
        dw.free()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want = matmul_bf16(x, w)
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    bound = 2 * k * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(wf).astype(np.float64).T)
    assert np.all(np.abs(a.astype(np.float64) - want) <= bound), np.abs(a - want).max()
