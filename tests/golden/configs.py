"""The benchmark configurations as scenarios, at the sizes the oracle finishes in
seconds (configuration 1 at full size; 2-5 shrunk, same shapes of work).

One driver runs each scenario against any (cache, backend) pair: the oracle cache
and the oracle backend to make the fixtures (make_golden.py), the shipped allocator
with the oracle backend on the CPU, and the shipped allocator with the HIP backend on
the GPU. Inputs are regenerated from their seeds (oracle.attn.normal); the fixtures
hold the outputs and a checksum of the inputs.

Backend protocol: begin_pass(pos, slot, pt_off, pages); store(layer, k, v) for the
pass rows; attend(layer, q, hq, window) -> [rows, hq*128]; copy_pages([(src, dst)]);
read_pages(layer, pages) -> (K bits, V bits) in [n][hkv][page][128].
"""

from __future__ import annotations

import numpy as np

from oracle.attn import OracleArena, normal
from oracle.kv_oracle import OracleKvCache

D = 128
SEED = 0x59415855


class OracleBackend:
    """The CPU oracle arena behind the backend protocol (f16 or f32 storage)."""

    def __init__(self, layers, pages, page, hkv, f16=True):
        self.arenas = [OracleArena(pages, page, hkv, D, f16=f16) for _ in range(layers)]
        self.page, self.hkv, self.f16 = page, hkv, f16

    def begin_pass(self, pos, slot, pt_off, pages):
        self.meta = (np.asarray(pos, np.uint32), np.asarray(slot, np.uint32),
                     np.asarray(pt_off, np.uint32), np.asarray(pages, np.uint32))

    def store(self, layer, k, v):
        self.arenas[layer].store(self.meta[1], k.reshape(len(self.meta[0]), -1),
                                 v.reshape(len(self.meta[0]), -1))

    def attend(self, layer, q, hq, window):
        pos, _, off, pages = self.meta
        return self.arenas[layer].attend(q, hq, pos, off, pages, window=window or 0)

    def copy_pages(self, copies):
        for s, d in copies:
            for a in self.arenas:
                a.copy_page(s, d)

    def read_pages(self, layer, pages):
        ks, vs = zip(*[self.arenas[layer].page_bits(int(p)) for p in pages])
        return np.stack(ks), np.stack(vs)


def _meta(pr):
    """(pos, slot, pt_off, pages) of an append result: oracle tuple or PassRows."""
    if isinstance(pr, tuple):
        _, pos, slot, off, pages, _ = pr
    else:
        m = pr.meta
        pos, slot, off, pages = m.pos, m.kv_slot, m.pt_off, m.pages
    return [np.asarray(x, np.uint32) for x in (pos, slot, off, pages)]


def _copies(c):
    return [(int(x[0]), int(x[1])) if isinstance(x, tuple) else (int(x.src), int(x.dst)) for x in c]


class Run:
    def __init__(self, cache, be, hkv, layers):
        self.cache, self.be, self.hkv, self.layers = cache, be, hkv, layers
        self.offset = 0
        self.inputs_sum = np.uint64(0)
        self.out = {}

    def draw(self, n):
        x = normal(n, SEED, self.offset)
        self.offset += n
        with np.errstate(over="ignore"):
            self.inputs_sum = np.uint64(self.inputs_sum + x.view(np.uint32).astype(np.uint64).sum())
        return x

    def copy(self, copies):
        cp = _copies(copies)
        if cp:
            self.be.copy_pages(cp)
        return cp

    def pass_(self, items, q_rows_hq=None, windows=None, keep=None):
        """Append items [(seq, ntokens)], store K/V in every layer, optionally attend."""
        copies = []
        try:
            pr = self.cache.append([(s, [7] * n) for s, n in items], copies)
        finally:
            cp = self.copy(copies)
        pos, slot, off, pages = _meta(pr)
        self.be.begin_pass(pos, slot, off, pages)
        rows = len(pos)
        outs = []
        for layer in range(self.layers):
            k = self.draw(rows * self.hkv * D).reshape(rows, self.hkv, D)
            v = self.draw(rows * self.hkv * D).reshape(rows, self.hkv, D)
            if q_rows_hq is None:
                self.be.store(layer, k, v)
                continue
            q = self.draw(rows * q_rows_hq * D).reshape(rows, q_rows_hq * D)
            w = windows[layer] if windows else 0
            outs.append(self.be.attend_append(layer, k, v, q, q_rows_hq, w)
                        if hasattr(self.be, "attend_append") else
                        (self.be.store(layer, k, v), self.be.attend(layer, q, q_rows_hq, w))[1])
        if keep is not None:
            self.out[keep + "_pos"], self.out[keep + "_slot"] = pos, slot
            self.out[keep + "_pt_off"], self.out[keep + "_pages"] = off, pages
            self.out[keep + "_copies"] = np.asarray(cp, np.uint32).reshape(-1, 2)
            for layer, o in enumerate(outs):
                self.out[f"{keep}_attn{layer}"] = np.asarray(o, np.float32)
            # The pages this pass wrote into, as stored (bit-exact comparison).
            written = np.unique(slot // self.be.page).astype(np.uint32)
            k, v = self.be.read_pages(0, written)
            self.out[keep + "_kv_pages"] = written
            self.out[keep + "_k_bits"] = np.asarray(k)
            self.out[keep + "_v_bits"] = np.asarray(v)
        return pos

    def prefill(self, lens, chunk=512):
        left = dict(lens)
        while any(n > 0 for n in left.values()):
            items, budget = [], chunk
            for s, n in left.items():
                if n > 0 and budget > 0:
                    t = min(n, budget)
                    items.append((s, t))
                    budget -= t
            for s, t in items:
                left[s] -= t
            self.pass_(items)


def scatter(cache, pages, page, seed):
    """Take the pool's pages out of the free list in a seeded order: allocate every
    page, then free them in a permuted order (the free list is a LIFO stack)."""
    from yaxus_amd.data import permutation

    holders = [cache.new_seq() for _ in range(pages)]
    for s in holders:
        cache.append([(s, [0] * page)], [])
    for i in permutation(pages, seed):
        cache.free_seq(holders[int(i)])


# (name, page, pool pages, layers, hq, hkv, f16)
CONFIGS = {
    "cfg1_decode_f32": dict(page=16, pages=256, layers=1, hq=16, hkv=4, f16=False),
    "cfg2_prefix_decode": dict(page=16, pages=160, layers=2, hq=16, hkv=4, f16=True),
    "cfg3_chunked_prefill": dict(page=16, pages=96, layers=1, hq=16, hkv=4, f16=True),
    "cfg4_long_sliding": dict(page=16, pages=1024, layers=4, hq=16, hkv=4, f16=True),
    "cfg5_verify_fork": dict(page=16, pages=160, layers=1, hq=16, hkv=4, f16=True),
}


def run_config(name, cache, be):
    """Runs configuration `name`; returns the outputs to compare (dict of arrays)."""
    c = CONFIGS[name]
    P = c["page"]
    r = Run(cache, be, c["hkv"], c["layers"])
    hq = c["hq"]
    if name == "cfg1_decode_f32":
        # 512 tokens in 32 pages from a 256-page pool in seeded order, append 1, attend.
        scatter(cache, c["pages"], P, SEED)
        s = cache.new_seq()
        r.prefill({s: 512})
        r.pass_([(s, 1)], q_rows_hq=hq, keep="step")
    elif name == "cfg2_prefix_decode":
        # 4 requests share a 64-token prefix (4 refcounted pages); own suffixes of
        # seeded length in [32, 192]; one decode step in 2 layers.
        scatter(cache, c["pages"], P, SEED + 2)
        base = cache.new_seq()
        r.prefill({base: 64})
        lens = [int(x) for x in 32 + (np.arange(4) * 37 + 11) % 161]
        seqs = [cache.fork(base, 64, []) for _ in range(4)]
        r.prefill(dict(zip(seqs, lens)))
        r.out["prefix_refs"] = np.array([cache.page_refs(p) if hasattr(cache, "page_refs")
                                         else cache.pool.refs[p] for p in cache.seq_pages(base)],
                                        np.uint32)
        r.pass_([(s, 1) for s in seqs], q_rows_hq=hq, keep="step")
    elif name == "cfg3_chunked_prefill":
        # 4 requests append a 32-row chunk on contexts of 8 mod 16 tokens (a half-filled
        # tail page); causal within the chunk plus everything before it.
        scatter(cache, c["pages"], P, SEED + 3)
        seqs = [cache.new_seq() for _ in range(4)]
        ctx = [8, 24, 104, 56]
        r.prefill(dict(zip(seqs, ctx)))
        r.pass_([(s, 32) for s in seqs], q_rows_hq=hq, keep="step")
    elif name == "cfg4_long_sliding":
        # 2 requests of 1024 tokens over a scattered 1024-page pool; layer 0 full,
        # layers 1-3 sliding (window 256); one decode step.
        scatter(cache, c["pages"], P, SEED + 4)
        seqs = [cache.new_seq() for _ in range(2)]
        r.prefill(dict(zip(seqs, [1023, 1023])))
        r.pass_([(s, 1) for s in seqs], q_rows_hq=hq, windows=[0, 256, 256, 256], keep="step")
    elif name == "cfg5_verify_fork":
        # 4 requests of 256 tokens, the first 128 shared; each verifies 5 draft tokens
        # (5 causal rows); then 2 requests fork from a partly filled tail page (copy on
        # write) and all roll back a seeded number of tokens in [0, 5].
        scatter(cache, c["pages"], P, SEED + 5)
        base = cache.new_seq()
        r.prefill({base: 128})
        seqs = [cache.fork(base, 128, []) for _ in range(4)]
        r.prefill(dict(zip(seqs, [128, 128, 127, 121])))
        r.pass_([(s, 5) for s in seqs], q_rows_hq=hq, keep="verify")
        forks = []
        for s in seqs[:2]:
            cp = []
            f = cache.fork(s, cache.seq_len(s) - 3, cp)
            r.out[f"fork{len(forks)}_copies"] = np.asarray(r.copy(cp), np.uint32).reshape(-1, 2)
            forks.append(f)
        for i, s in enumerate(seqs + forks):
            back = (i * 3 + 2) % 6
            cache.truncate(s, cache.seq_len(s) - back)
        r.out["after_pages"] = np.concatenate([np.asarray(cache.seq_pages(s), np.uint32)
                                               for s in seqs + forks])
        r.out["after_lens"] = np.array([cache.seq_len(s) for s in seqs + forks], np.uint32)
        # One more decode step on every sequence after the rollback.
        r.pass_([(s, 1) for s in seqs + forks], q_rows_hq=hq, keep="step")
    r.out["inputs_sum"] = np.array([r.inputs_sum], np.uint64)
    r.out["free_pages"] = np.array([cache.free_pages()], np.uint32)
    return r.out


def oracle_pair(name):
    c = CONFIGS[name]
    return (OracleKvCache(c["pages"], 1 << 20, c["page"]),
            OracleBackend(c["layers"], c["pages"], c["page"], c["hkv"], f16=c["f16"]))
