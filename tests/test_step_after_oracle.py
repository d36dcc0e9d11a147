"""The oracle of the step after attention (oracle/attn_oracle.c: orc_matmul_bf16,
orc_argmax), pinned without the reference's code: an f64 brute force and exact known
answers for the matmul (including inputs where the 16-lane order of dot_bf16,
crates/yaxus-backend-cpu/src/lib.rs:234-248, decides the result), and the argmax's
rule (lib.rs:432-440) on ties, NaN, infinities and signed zeros, and against numpy."""

import numpy as np

from oracle.attn import argmax_rows, matmul_bf16


def _bf16_bits(a):
    """Round f32 to bf16 bits (nearest even)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def _bf16_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_matmul_against_f64_brute_force():
    rng = np.random.default_rng(1)
    for t, k, n in [(1, 2048, 64), (3, 40, 17), (5, 128, 33), (16, 1000, 8)]:
        x = rng.standard_normal((t, k), dtype=np.float32)
        w = _bf16_bits(rng.standard_normal((n, k), dtype=np.float32))
        got = matmul_bf16(x, w)
        exact = x.astype(np.float64) @ _bf16_f32(w).astype(np.float64).T
        bound = k * 2.0 ** -23 * (np.abs(x).astype(np.float64) @ np.abs(_bf16_f32(w)).astype(np.float64).T)
        assert np.all(np.abs(got - exact) <= bound + 1e-30)


def test_matmul_known_answers():
    one = 0x3F80  # bf16 1.0
    # One-hot weight rows pick entries of x exactly.
    x = np.arange(48, dtype=np.float32).reshape(2, 24) * 0.37
    w = np.zeros((3, 24), np.uint16)
    w[0, 5] = w[1, 23] = w[2, 0] = one
    np.testing.assert_array_equal(matmul_bf16(x, w), x[:, [5, 23, 0]])
    # Lane 0 holds 1e8 (k = 0) and -1e8 (k = 16): they cancel inside the lane before the
    # ones of lanes 1..15 are added, so the 16-lane order gives exactly 15; a single
    # running sum would lose the ones against 1e8 and give 8 (or other values).
    x = np.ones((1, 32), np.float32)
    x[0, 0], x[0, 16] = 1e8, -1e8
    x[0, 17:] = 0
    w = np.full((1, 32), one, np.uint16)
    assert matmul_bf16(x, w)[0, 0] == 15.0
    # The lanes are then summed in order: 1e8, fourteen ones (each lost against 1e8),
    # then -1e8: exactly 0 (any other order keeps some of the ones).
    x = np.ones((1, 16), np.float32)
    x[0, 0], x[0, 15] = 1e8, -1e8
    assert matmul_bf16(x, np.full((1, 16), one, np.uint16))[0, 0] == 0.0
    # Past the last whole chunk the rest is added one by one after the lane sum.
    x = np.zeros((1, 18), np.float32)
    x[0, 0], x[0, 16], x[0, 17] = 1e8, 1.0, -1e8
    assert matmul_bf16(x, np.full((1, 18), one, np.uint16))[0, 0] == 0.0


def test_argmax_rule():
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rows = np.array([
        [1, 3, 3, 2],            # ties: the first
        [nan, 1, nan, 0],        # NaN never wins
        [nan, nan, nan, nan],    # nothing above -inf: index 0
        [-inf, -inf, -inf, -inf],
        [-inf, -5, -inf, -5],
        [-0.0, 0.0, 0.0, -1],    # -0 and +0 are equal: the first
        [1, inf, 2, inf],
        [-1, -2, -3, -0.5],
    ], dtype=np.float32)
    np.testing.assert_array_equal(argmax_rows(rows), [1, 1, 0, 0, 1, 0, 1, 3])


def test_argmax_against_numpy():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((20, 5000), dtype=np.float32)
    a[3, [7, 4000]] = 50.0  # a tie at the maximum
    np.testing.assert_array_equal(argmax_rows(a), np.argmax(a, axis=1))
