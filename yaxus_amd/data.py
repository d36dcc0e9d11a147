"""Synthetic inputs of the benchmark configurations.

N(0,1) values from splitmix64 -> Box-Muller: pair k of stream ``seed`` draws
``u1 = splitmix64(seed + 2k) >> 11`` and ``u2 = splitmix64(seed + 2k + 1) >> 11``
(53-bit fractions), ``r = sqrt(-2 ln(1 - u1))``, ``th = 2 pi u2``; element 2k is
``r cos th`` and element 2k+1 is ``r sin th``, computed in f64 and rounded to f32
(then to f16 where the arena stores f16). The device fill kernel (``yx_fill_normal``)
draws the same stream; parity tests upload host-drawn values instead, so their
inputs are bit-identical on both sides.
"""

from __future__ import annotations

import numpy as np

SEED = 0x59415855  # the configurations' seed

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x):
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def normal(n, seed=SEED, offset=0):
    """``n`` f32 values of stream ``seed`` starting at element ``offset``."""
    e = np.arange(offset, offset + n, dtype=np.uint64)
    k = e >> np.uint64(1)
    with np.errstate(over="ignore"):
        a = splitmix64(np.uint64(seed) + np.uint64(2) * k)
        b = splitmix64(np.uint64(seed) + np.uint64(2) * k + np.uint64(1))
    u1 = (a >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    th = 6.283185307179586 * u2
    odd = (e & np.uint64(1)).astype(bool)
    return np.where(odd, r * np.sin(th), r * np.cos(th)).astype(np.float32)


def uniform_ints(n, lo, hi, seed=SEED, offset=0):
    """``n`` integers uniform in ``[lo, hi]`` (inclusive) from splitmix64."""
    e = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = splitmix64(np.uint64(seed) ^ np.uint64(0xA5A5A5A5) + e)
    span = np.uint64(hi - lo + 1)
    return (lo + (z % span).astype(np.int64)).astype(np.int64)


def permutation(n, seed=SEED):
    """A seeded permutation of ``range(n)`` (Fisher-Yates over splitmix64 draws)."""
    perm = np.arange(n, dtype=np.int64)
    z = splitmix64(np.uint64(seed) + np.arange(n, dtype=np.uint64) * np.uint64(7919))
    for i in range(n - 1, 0, -1):
        j = int(z[i] % np.uint64(i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    return perm
