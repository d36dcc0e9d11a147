"""The RoPE table the q/k step reads, built on the host as the model builds it.

Restates `Rope::new` for the default scaling and `Rope::cos_sin`
(crates/yaxus-model/src/config.rs:187-219): inverse frequencies in f32, the angle
`pos * inv_freq` in f32, cos and sin in f64, rounded to f32 and multiplied by the
concentration in f32. The table is `[2][max_pos][dim / 2]`: cos, then sin, the layout
the reference GPU backend uploads per layer kind (crates/yaxus-backend-gpu/src/ops/
attention.rs:112-120) and `yx_qk_rope_append_dev` reads.
"""

from __future__ import annotations

import numpy as np


def inv_freq(dim, theta):
    """`Rope::new` with default scaling: 1 / theta^(i / dim) for even i, in f32."""
    i = np.arange(0, dim, 2, dtype=np.float32)
    freq = np.power(np.float32(theta), i / np.float32(dim), dtype=np.float32)
    return (np.float32(1.0) / freq).astype(np.float32)


def rope_table(inv_freq_, concentration, max_pos):
    """cos/sin of every position below max_pos: float32 `[2][max_pos][len(inv_freq)]`."""
    f = np.asarray(inv_freq_, np.float32)
    pos = np.arange(max_pos, dtype=np.float32)[:, None]
    a = (pos * f[None, :]).astype(np.float32)
    c = np.float32(concentration)
    out = np.empty((2, max_pos, f.size), np.float32)
    out[0] = np.cos(a.astype(np.float64)).astype(np.float32) * c
    out[1] = np.sin(a.astype(np.float64)).astype(np.float32) * c
    return out
