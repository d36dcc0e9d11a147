"""Builds paged-attention scenarios shared by the GPU tests and the smoke check.

A scenario runs the product allocator (KvCache) to lay sequences out in pages, writes
the same K/V rows into the device arena (through the append kernel) and into the
oracle's slot-major arena, then forms the pass to check.
"""

from __future__ import annotations

import numpy as np

from oracle.attn import OracleArena
from yaxus_amd import KvCache
from oracle.attn import normal

D = 128


class Scenario:
    def __init__(self, hip, pages, page, hkv, layers=1, seed=1234, pool_seed=None, f32=False):
        self.hip, self.page, self.hkv = hip, page, hkv
        self.cache = KvCache(pages, 1 << 30, page)
        self.kv = hip.new_kv(layers, pages, page, hkv, f32=f32)
        self.orc = [OracleArena(pages, page, hkv, D, f16=not f32) for _ in range(layers)]
        self.layers = layers
        self.seed = seed
        self.offset = 0
        if pool_seed is not None:
            # Scatter pages: take them out of the free list in a seeded order by
            # allocating all, then freeing in a permuted order (LIFO reuse).
            rng = np.random.default_rng(pool_seed)
            ids = [self.cache.new_seq() for _ in range(pages)]
            for s in ids:
                self.cache.append([(s, [0] * page)], [])
            for i in rng.permutation(pages):
                self.cache.free_seq(ids[i])

    def draw(self, n):
        x = normal(n, self.seed, self.offset)
        self.offset += n
        return x

    def run_pass(self, items, copies=None):
        """Appends ``items`` = [(seq, ntokens)] to the cache and returns PassRows."""
        cp = [] if copies is None else copies
        pr = self.cache.append([(s, [7] * n) for s, n in items], cp)
        self.hip.copy_pages(self.kv, cp)
        for c in cp:
            for o in self.orc:
                o.copy_page(c.src, c.dst)
        self.hip.begin_pass(pr.meta)
        return pr

    def store(self, pr, layer=0):
        """Draws K/V for the pass rows and writes them on both sides."""
        rows = len(pr.meta.pos)
        k = self.draw(rows * self.hkv * D).reshape(rows, self.hkv, D)
        v = self.draw(rows * self.hkv * D).reshape(rows, self.hkv, D)
        self.hip.append(self.kv, layer, k, v)
        self.orc[layer].store(pr.meta.kv_slot, k.reshape(rows, -1), v.reshape(rows, -1))
        return k, v

    def prefill(self, seqs_lens, chunk=512):
        """Appends tokens to sequences in passes of at most ``chunk`` rows, storing K/V."""
        left = dict(seqs_lens)
        while any(v > 0 for v in left.values()):
            items, budget = [], chunk
            for s, n in left.items():
                if n > 0 and budget > 0:
                    t = min(n, budget)
                    items.append((s, t))
                    budget -= t
            for s, t in items:
                left[s] -= t
            pr = self.run_pass(items)
            for layer in range(self.layers):
                self.store(pr, layer)


def close(a, b, atol=2e-3, rtol=1e-3):
    """The path's tolerance for f16 KV with f32 accumulation."""
    return np.abs(a - b) <= atol + rtol * np.abs(b)
