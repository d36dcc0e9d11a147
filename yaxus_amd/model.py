"""The forward-pass order of the paged path: ``Model``'s KV half.

Mirrors the parts of ``yaxus_model::Model`` (crates/yaxus-model/src/lib.rs:256-471)
that touch the KV cache: ``begin`` / ``start`` / ``prefill`` / ``forward`` / ``finish``
/ ``fork`` / ``truncate`` and the page copies an operation asks for, which are made
before the next pass even when the operation fails (kv.rs:4-7, lib.rs:349-353, 441-444).
The weight products around attention are out of scope: ``forward`` takes, per layer,
the rows' inputs from a caller-supplied function and runs the layer's attention
through the backend (``HipBackend`` on a GPU; any object with the same methods, such
as the do-nothing backend of the tests, otherwise). The inputs are either a
``LayerQkv`` (the projected rows and the layer's norm weights and RoPE table:
``Backend::attention`` in full, write_rows then attend) or ``(k, v, q)`` already
normalised and rotated (the K/V store and attend only).
"""

from __future__ import annotations

from typing import NamedTuple

from .kv import KvCache, KvError

DEFAULT_KV_TOKENS = 16384  # lib.rs:238
DEFAULT_MAX_POS = 8192  # lib.rs:239


class LayerQkv(NamedTuple):
    """One layer's attention inputs as ``Backend::attention`` takes them (lib.rs:132):
    qkv ``[rows][(hq + 2 hkv) * d]``, q_norm/k_norm ``[d]``, the RoPE table of the
    layer's kind (``rope.rope_table``) and the RMSNorm eps."""

    qkv: object
    q_norm: object
    k_norm: object
    rope_cs: object
    eps: float


class ModelError(Exception):
    """An ``Err`` of ``Model`` itself (empty pass, chunk size)."""


class PagedModel:
    """``layers`` attention layers over one paged arena of ``pages`` pages."""

    def __init__(self, backend, pages, max_pos=DEFAULT_MAX_POS, page=128, layers=1, hkv=1,
                 hq=1, windows=None, chunk=512, prefix_cache=True, kv=None):
        self.backend = backend
        self.page, self.layers, self.hkv, self.hq = page, layers, hkv, hq
        self.windows = list(windows) if windows is not None else [None] * layers
        self.chunk = chunk  # lib.rs:325: rows per forward pass at most
        self.kv = kv if kv is not None else backend.new_kv(layers, pages, page, hkv)
        self.seqs = KvCache(pages, max_pos, page)
        self.seqs.set_prefix_reuse(prefix_cache)

    # lib.rs:349-353
    def _copy_pages(self, copies):
        if copies:
            self.backend.copy_pages(self.kv, copies)

    def set_prefix_cache(self, on):
        self.seqs.set_prefix_reuse(on)

    def clear_prefix_cache(self):
        self.seqs.clear_prefix_cache()

    def new_seq(self):
        return self.seqs.new_seq()

    def free_seq(self, sid):
        self.seqs.free_seq(sid)

    # lib.rs:374-379
    def begin(self, prompt):
        copies = []
        try:
            return self.seqs.begin(prompt, copies)
        finally:
            self._copy_pages(copies)

    # lib.rs:383-393
    def start(self, prompt, layer_inputs=None):
        sid, reused = self.begin(prompt)
        try:
            out = self.prefill(sid, prompt[reused:], layer_inputs)
        except Exception:
            self.free_seq(sid)
            raise
        return sid, out

    def finish(self, sid):
        self.seqs.finish(sid)

    def seq_len(self, sid):
        return self.seqs.seq_len(sid)

    def seq_tokens(self, sid):
        return self.seqs.seq_tokens(sid)

    def truncate(self, sid, n):
        self.seqs.truncate(sid, n)

    # lib.rs:423-429
    def fork(self, sid, n):
        copies = []
        try:
            return self.seqs.fork(sid, n, copies)
        finally:
            self._copy_pages(copies)

    def free_pages(self):
        return self.seqs.free_pages()

    def arena(self):
        return self.seqs.total_pages(), self.seqs.max_pos()

    # lib.rs:434-471 (the KV half): append -> copy pages -> begin_pass -> per layer
    # store K/V + attend. Returns (PassRows, per-layer attention outputs).
    def forward(self, items, layer_inputs=None):
        rows = sum(len(t) for _, t in items)
        if rows == 0:
            raise ModelError("empty pass")
        if rows > self.chunk:
            raise ModelError(f"pass of {rows} rows exceeds the chunk size {self.chunk}")
        copies = []
        try:
            pr = self.seqs.append(items, copies)
        finally:
            self._copy_pages(copies)
        self.backend.begin_pass(pr.meta)
        outs = []
        for layer in range(self.layers):
            if layer_inputs is None:
                outs.append(None)
                continue
            inp = layer_inputs(layer, pr.meta)
            if isinstance(inp, LayerQkv):
                outs.append(self.backend.attention(self.kv, layer, inp.qkv, inp.q_norm,
                                                   inp.k_norm, inp.rope_cs, inp.eps, self.hq,
                                                   window=self.windows[layer]))
                continue
            k, v, q = inp
            outs.append(self.backend.attend_append(self.kv, layer, k, v, q, self.hq,
                                                   window=self.windows[layer]))
        return pr, outs

    # lib.rs:475-484
    def prefill(self, sid, ids, layer_inputs=None):
        if len(ids) == 0:
            raise ModelError("empty input")
        out = None
        for i in range(0, len(ids), self.chunk):
            out = self.forward([(sid, ids[i:i + self.chunk])], layer_inputs)
        return out


__all__ = ["PagedModel", "LayerQkv", "ModelError", "KvError", "DEFAULT_KV_TOKENS", "DEFAULT_MAX_POS"]
