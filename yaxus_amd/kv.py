"""Host-side paged KV bookkeeping: ``KvCache`` over the native allocator.

Mirrors ``yaxus_model::kv::KvCache`` (crates/yaxus-model/src/kv.rs:110-353) method for
method; the page size is a constructor argument (the reference fixes ``PAGE = 128``,
kv.rs:17). Operations that need pages copied append ``PageCopy`` values to the
``copies`` list passed in, whether or not they then succeed (kv.rs:4-7), like the
reference's ``&mut Vec<PageCopy>`` argument. Errors the reference returns as ``Err``
raise ``KvError``; ``truncate`` beyond the end (a reference panic) raises it too.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import YxError

MIN_REUSE = 16  # kv.rs:25
MAX_CACHED = 32  # kv.rs:27


class KvError(YxError):
    pass


@dataclass(frozen=True)
class PageCopy:
    """kv.rs:35-38: page ``src`` is copied to ``dst`` in every layer."""

    src: int
    dst: int


@dataclass
class PassMeta:
    """lib.rs:63-89: row metadata of one forward pass (the gather indices)."""

    ids: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    pos: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    kv_slot: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    pt_off: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    pages: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))

    def page_table(self, row):
        return self.pages[int(self.pt_off[row]):]

    def slot(self, row, pos, page):
        return int(self.page_table(row)[pos // page]) * page + pos % page


@dataclass
class PassRows:
    """kv.rs:121-124: the pass metadata and the row of each item's last token."""

    meta: PassMeta
    last: list


class SeqId(int):
    """kv.rs:31: identifies a sequence in a cache."""


class KvCache:
    """kv.rs:110-353 on the native allocator (yaxus_amd/csrc/kv_cache.cpp)."""

    def __init__(self, pages, max_pos, page=128):
        self._L = _lib.kv_lib()
        h = ctypes.c_void_p()
        self._check(self._L.yx_cache_create(pages, max_pos, page, ctypes.byref(h)))
        self._h = h
        self.page = page

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._L.yx_cache_destroy(h)
            self._h = None

    def _check(self, rc):
        if rc != _lib.YX_OK:
            raise KvError(rc, self._L.yx_cache_last_error().decode())

    def _drain(self, copies):
        n = self._L.yx_cache_pending_copies(self._h)
        if n == 0:
            return
        buf = np.zeros(2 * n, np.uint32)
        got = self._L.yx_cache_take_copies(self._h, _lib.ptr(buf), n)
        if copies is not None:
            copies.extend(PageCopy(int(buf[2 * i]), int(buf[2 * i + 1])) for i in range(got))

    # kv.rs:140
    def set_prefix_reuse(self, on):
        self._L.yx_cache_set_prefix_reuse(self._h, 1 if on else 0)

    # kv.rs:154
    def new_seq(self):
        return SeqId(self._L.yx_cache_new_seq(self._h))

    # kv.rs:158
    def free_seq(self, sid):
        self._L.yx_cache_free_seq(self._h, int(sid))

    # kv.rs:181
    def clear_prefix_cache(self):
        self._L.yx_cache_clear_prefix_cache(self._h)

    # kv.rs:189
    def begin(self, prompt, copies):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        sid = ctypes.c_uint64()
        reused = ctypes.c_size_t()
        rc = self._L.yx_cache_begin(self._h, _lib.ptr(p), len(p), ctypes.byref(sid),
                                    ctypes.byref(reused))
        self._drain(copies)
        self._check(rc)
        return SeqId(sid.value), reused.value

    # kv.rs:231
    def finish(self, sid):
        self._L.yx_cache_finish(self._h, int(sid))

    # kv.rs:240
    def seq_len(self, sid):
        return self._L.yx_cache_seq_len(self._h, int(sid))

    # kv.rs:245
    def seq_tokens(self, sid):
        n = self.seq_len(sid)
        out = np.zeros(max(n, 1), np.uint32)
        self._L.yx_cache_seq_tokens(self._h, int(sid), _lib.ptr(out), n)
        return [int(x) for x in out[:n]]

    def seq_pages(self, sid):
        n = self._L.yx_cache_seq_pages(self._h, int(sid), None, 0)
        out = np.zeros(max(n, 1), np.uint32)
        self._L.yx_cache_seq_pages(self._h, int(sid), _lib.ptr(out), n)
        return [int(x) for x in out[:n]]

    # kv.rs:250-262
    def free_pages(self):
        return self._L.yx_cache_free_pages(self._h)

    def total_pages(self):
        return self._L.yx_cache_total_pages(self._h)

    def max_pos(self):
        return self._L.yx_cache_max_pos(self._h)

    def page_refs(self, page):
        return self._L.yx_cache_page_refs(self._h, page)

    # kv.rs:265
    def truncate(self, sid, n):
        self._check(self._L.yx_cache_truncate(self._h, int(sid), n))

    # kv.rs:277
    def fork(self, sid, n, copies):
        out = ctypes.c_uint64()
        rc = self._L.yx_cache_fork(self._h, int(sid), n, ctypes.byref(out))
        self._drain(copies)
        self._check(rc)
        return SeqId(out.value)

    # kv.rs:330
    def append(self, items, copies):
        """``items`` = [(seq, tokens)]; returns ``PassRows``."""
        ids = np.array([int(s) for s, _ in items], dtype=np.uint64)
        counts = np.array([len(t) for _, t in items], dtype=np.uintp)
        toks = np.ascontiguousarray(
            np.concatenate([np.asarray(t, dtype=np.uint32) for _, t in items])
            if items else np.zeros(0, np.uint32), dtype=np.uint32)
        rc = self._L.yx_cache_append(self._h, len(items), _lib.ptr(ids), _lib.ptr(counts),
                                     _lib.ptr(toks) if len(toks) else None)
        self._drain(copies)
        self._check(rc)
        rows = self._L.yx_cache_pass_rows(self._h)
        npg = self._L.yx_cache_pass_npages(self._h)
        nit = self._L.yx_cache_pass_nitems(self._h)
        m = PassMeta(*(np.zeros(rows, np.uint32) for _ in range(4)), np.zeros(npg, np.uint32))
        last = np.zeros(nit, np.uintp)
        self._L.yx_cache_pass_get(self._h, _lib.ptr(m.ids), _lib.ptr(m.pos), _lib.ptr(m.kv_slot),
                                  _lib.ptr(m.pt_off), _lib.ptr(m.pages), _lib.ptr(last))
        return PassRows(m, [int(x) for x in last])
