"""The host RoPE table (yaxus_amd.rope) against the oracle's Rope::cos_sin restatement
(crates/yaxus-model/src/config.rs:213-219) and against what the functions must be."""

import numpy as np

from oracle.attn import cos_sin_table
from yaxus_amd.rope import inv_freq, rope_table


def test_table_bits_equal_the_oracle():
    f = inv_freq(128, 10000.0)
    for conc, n in [(1.0, 4096), (1.2079441, 40000)]:
        a, b = rope_table(f, conc, n), cos_sin_table(f, conc, n)
        assert a.shape == b.shape == (2, n, 64)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_table_closed_forms():
    f = inv_freq(128, 10000.0)
    assert f[0] == 1.0 and np.all(np.diff(f) < 0)  # theta^0, then decreasing
    t = rope_table(f, 1.0, 3000)
    assert np.all(t[0, 0] == 1.0) and np.all(t[1, 0] == 0.0)  # position 0: no rotation
    # Position 1, first pair: the angle is exactly 1 radian.
    assert t[0, 1, 0] == np.float32(np.cos(1.0)) and t[1, 1, 0] == np.float32(np.sin(1.0))
    # cos^2 + sin^2 = 1 to f32 rounding, and the concentration scales both.
    assert np.abs(t[0] ** 2 + t[1] ** 2 - 1.0).max() < 1e-6
    c = rope_table(f, 1.5, 100)
    assert np.allclose(c, rope_table(f, 1.0, 100) * np.float32(1.5), rtol=1e-7, atol=0)
