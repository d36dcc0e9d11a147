"""The HIP backend of the KV path: the part of yaxus's ``Backend`` trait that touches
the KV arena (crates/yaxus-model/src/lib.rs:95-171), over ``libyaxus_hip.so``.

    Backend::new_kv      (lib.rs:118)  -> HipBackend.new_kv
    Backend::copy_page   (lib.rs:120)  -> HipBackend.copy_page / copy_pages
    Backend::begin_pass  (lib.rs:123)  -> HipBackend.begin_pass
    Backend::attention   (lib.rs:132)  -> HipBackend.append (the K/V store of
                                          write_rows) + HipBackend.attend

Tensors are ``DeviceTensor`` values (device memory owned by the context); numpy arrays
are accepted where a host round trip is intended. A missing library, or a context
that cannot open a gfx950 device, raises: nothing here computes on the host.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check_hip, ptr


def _need(t, nbytes, what):
    """Raises unless device tensor t holds at least nbytes: the kernels take plain
    pointers, so a short buffer would be read or written past its end."""
    if t.nbytes < nbytes:
        raise ValueError(f"{what}: device tensor of {t.nbytes} bytes, {nbytes} needed")


class DeviceTensor:
    """A device buffer of a fixed numpy dtype and shape, freed with its context."""

    def __init__(self, backend, shape, dtype):
        self.backend = backend
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check_hip(backend.L.yx_dev_alloc(backend.ctx, max(self.nbytes, 16), ctypes.byref(p)))
        self.ptr = p

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError(f"upload of {a.nbytes} bytes into {self.nbytes}")
        check_hip(self.backend.L.yx_memcpy_h2d(self.backend.ctx, self.ptr, ptr(a), self.nbytes))
        return self

    def numpy(self):
        out = np.empty(self.shape, dtype=self.dtype)
        check_hip(self.backend.L.yx_memcpy_d2h(self.backend.ctx, ptr(out), self.ptr, self.nbytes))
        return out

    def free(self):
        if self.ptr:
            self.backend.L.yx_dev_free(self.backend.ctx, self.ptr)
            self.ptr = None


class Kv:
    """The arena of one model: ``layers`` layers of ``pages`` pages (binary16 K/V, or
    f32 with ``f32=True``)."""

    def __init__(self, backend, handle, layers, pages, page, hkv, d, f32=False):
        self.backend, self.h = backend, handle
        self.layers, self.pages, self.page, self.hkv, self.d = layers, pages, page, hkv, d
        self.f32 = f32
        self.bits = np.uint32 if f32 else np.uint16

    def layer_ptr(self, layer, which):
        p = ctypes.c_void_p()
        check_hip(self.backend.L.yx_kv_layer_ptr(self.h, layer, which, ctypes.byref(p)))
        return p

    @property
    def page_bytes(self):
        return self.backend.L.yx_kv_page_bytes(self.h)

    def read_pages(self, layer, pages):
        """(K, V) bits of the pages, each ``[n][hkv][page][d]`` uint16 (uint32 for f32)."""
        pg = np.ascontiguousarray(pages, dtype=np.uint32)
        k = np.empty((len(pg), self.hkv, self.page, self.d), self.bits)
        v = np.empty_like(k)
        check_hip(self.backend.L.yx_kv_read_pages(self.backend.ctx, self.h, layer, ptr(pg),
                                                  len(pg), ptr(k), ptr(v)))
        return k, v

    def write_pages(self, layer, pages, k, v):
        pg = np.ascontiguousarray(pages, dtype=np.uint32)
        k, v = self._as_bits(k), self._as_bits(v)
        n = len(pg) * self.hkv * self.page * self.d
        if k.size != n or v.size != n:
            raise ValueError("k/v must be [n][hkv][page][d] of the arena's dtype")
        check_hip(self.backend.L.yx_kv_write_pages(self.backend.ctx, self.h, layer, ptr(pg),
                                                   len(pg), ptr(k), ptr(v)))

    def _as_bits(self, a):
        a = np.ascontiguousarray(a)
        return a.view(self.bits) if a.dtype.itemsize == np.dtype(self.bits).itemsize else a.astype(self.bits)

    def destroy(self):
        if self.h:
            self.backend.L.yx_kv_destroy(self.backend.ctx, self.h)
            self.h = None


class HipBackend:
    """One device context (one HIP stream) and the KV path's operations on it."""

    def __init__(self, device=0):
        self.L = _lib.hip_lib()
        c = ctypes.c_void_p()
        check_hip(self.L.yx_ctx_create(device, ctypes.byref(c)))
        self.ctx = c
        self.rows = 0

    def name(self):
        return "hip (gfx950)"

    def close(self):
        if self.ctx:
            self.L.yx_ctx_destroy(self.ctx)
            self.ctx = None

    def set_option(self, key, value):
        check_hip(self.L.yx_ctx_set_option(self.ctx, key.encode(), int(value)))

    def sync(self):
        check_hip(self.L.yx_sync(self.ctx))

    def tensor(self, shape, dtype=np.float32):
        return DeviceTensor(self, shape, dtype)

    # Backend::new_kv (lib.rs:118)
    def new_kv(self, layers, pages, page, hkv, d=128, f32=False):
        h = ctypes.c_void_p()
        check_hip(self.L.yx_kv_create(self.ctx, layers, pages, page, hkv, d,
                                      _lib.YX_DTYPE_F32 if f32 else _lib.YX_DTYPE_F16,
                                      ctypes.byref(h)))
        return Kv(self, h, layers, pages, page, hkv, d, f32)

    # Backend::copy_page (lib.rs:120), batched in list order
    def copy_pages(self, kv, copies):
        if not copies:
            return
        src = np.array([c.src for c in copies], np.uint32)
        dst = np.array([c.dst for c in copies], np.uint32)
        check_hip(self.L.yx_kv_copy_pages(self.ctx, kv.h, ptr(src), ptr(dst), len(src)))

    def copy_page(self, kv, src, dst):
        s = np.array([src], np.uint32)
        d = np.array([dst], np.uint32)
        check_hip(self.L.yx_kv_copy_pages(self.ctx, kv.h, ptr(s), ptr(d), 1))

    # Backend::begin_pass (lib.rs:123)
    def begin_pass(self, meta):
        pos = np.ascontiguousarray(meta.pos, np.uint32)
        slot = np.ascontiguousarray(meta.kv_slot, np.uint32)
        off = np.ascontiguousarray(meta.pt_off, np.uint32)
        pages = np.ascontiguousarray(meta.pages, np.uint32)
        check_hip(self.L.yx_pass_begin(self.ctx, len(pos), ptr(pos), ptr(slot), ptr(off),
                                       ptr(pages), len(pages)))
        self.rows = len(pos)
        self._keep = (pos, slot, off, pages)

    # The K/V store of Backend::attention (backend-cpu lib.rs:378-383)
    def append(self, kv, layer, k, v):
        if isinstance(k, DeviceTensor):
            _need(k, self.rows * kv.hkv * kv.d * 4, "k")
            _need(v, self.rows * kv.hkv * kv.d * 4, "v")
            check_hip(self.L.yx_kv_append_dev(self.ctx, kv.h, layer, k.ptr, v.ptr))
            return
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        if k.size != self.rows * kv.hkv * kv.d or v.size != k.size:
            raise ValueError("k/v must be [rows][hkv][head_dim] f32")
        check_hip(self.L.yx_kv_append(self.ctx, kv.h, layer, ptr(k), ptr(v)))

    # write_rows (backend-cpu lib.rs:359-385): q/k RMSNorm + RoPE of the pass's rows, K/V
    # stored at their slots; returns q. qkv `[rows][(hq + 2 hkv) * d]`, q_norm/k_norm
    # `[d]`, rope_cs from `rope.rope_table`. DeviceTensors stay on the device; numpy
    # arrays go through temporaries and q comes back as numpy.
    def qk_rope_append(self, kv, layer, qkv, q_norm, k_norm, rope_cs, eps, hq, out=None):
        rope_len = int(rope_cs.shape[1]) if len(rope_cs.shape) == 3 else int(rope_cs.shape[0]) // 2
        if isinstance(qkv, DeviceTensor):
            out = out if out is not None else self.tensor((self.rows, hq * kv.d))
            _need(qkv, self.rows * (hq + 2 * kv.hkv) * kv.d * 4, "qkv")
            _need(out, self.rows * hq * kv.d * 4, "q out")
            check_hip(self.L.yx_qk_rope_append_dev(self.ctx, kv.h, layer, qkv.ptr, q_norm.ptr,
                                                   k_norm.ptr, rope_cs.ptr, rope_len, float(eps),
                                                   hq, kv.hkv, out.ptr))
            return out
        qkv = np.ascontiguousarray(qkv, np.float32)
        if qkv.size != self.rows * (hq + 2 * kv.hkv) * kv.d:
            raise ValueError("qkv must be [rows][(hq + 2 hkv) * head_dim] f32")
        tmp = [self.tensor(a.shape) for a in (qkv, q_norm, k_norm, rope_cs)]
        try:
            for t, a in zip(tmp, (qkv, q_norm, k_norm, rope_cs)):
                t.upload(np.ascontiguousarray(a, np.float32))
            o = self.tensor((self.rows, hq * kv.d))
            try:
                self.qk_rope_append(kv, layer, tmp[0], tmp[1], tmp[2], tmp[3], eps, hq, out=o)
                return o.numpy()
            finally:
                o.free()
        finally:
            for t in tmp:
                t.free()

    # Backend::attention (lib.rs:132; backend-cpu lib.rs:516-530): write_rows, then attend
    # the rows' queries (one launch for decode passes). Device tensors stay on the
    # device (no synchronisation); numpy arrays go through temporaries.
    def attention(self, kv, layer, qkv, q_norm, k_norm, rope_cs, eps, hq, window=None,
                  scale=None, out=None):
        scale = float(np.float32(1.0) / np.sqrt(np.float32(kv.d))) if scale is None else scale
        w = int(window or 0)
        rope_len = int(rope_cs.shape[1]) if len(rope_cs.shape) == 3 else int(rope_cs.shape[0]) // 2
        if isinstance(qkv, DeviceTensor):
            out = out if out is not None else self.tensor((self.rows, hq * kv.d))
            _need(qkv, self.rows * (hq + 2 * kv.hkv) * kv.d * 4, "qkv")
            _need(out, self.rows * hq * kv.d * 4, "out")
            check_hip(self.L.yx_attention_qkv_dev(self.ctx, kv.h, layer, qkv.ptr, q_norm.ptr,
                                                  k_norm.ptr, rope_cs.ptr, rope_len, float(eps),
                                                  out.ptr, hq, kv.hkv, w, scale))
            return out
        qkv = np.ascontiguousarray(qkv, np.float32)
        if qkv.size != self.rows * (hq + 2 * kv.hkv) * kv.d:
            raise ValueError("qkv must be [rows][(hq + 2 hkv) * head_dim] f32")
        arrays = (qkv, q_norm, k_norm, rope_cs)
        tmp = [self.tensor(np.shape(a)) for a in arrays]
        try:
            for t, a in zip(tmp, arrays):
                t.upload(np.ascontiguousarray(a, np.float32))
            o = self.tensor((self.rows, hq * kv.d))
            try:
                self.attention(kv, layer, tmp[0], tmp[1], tmp[2], tmp[3], eps, hq, window=window,
                               scale=scale, out=o)
                return o.numpy()
            finally:
                o.free()
        finally:
            for t in tmp:
                t.free()

    # The attend half of Backend::attention (backend-cpu lib.rs:389-427)
    def attend(self, kv, layer, q, hq, window=None, scale=None, out=None):
        scale = float(np.float32(1.0) / np.sqrt(np.float32(kv.d))) if scale is None else scale
        w = int(window or 0)
        if isinstance(q, DeviceTensor):
            out = out if out is not None else self.tensor((self.rows, hq * kv.d))
            _need(q, self.rows * hq * kv.d * 4, "q")
            _need(out, self.rows * hq * kv.d * 4, "out")
            check_hip(self.L.yx_attention_dev(self.ctx, kv.h, layer, q.ptr, out.ptr, hq, kv.hkv,
                                              w, scale))
            return out
        q = np.ascontiguousarray(q, np.float32)
        if q.size != self.rows * hq * kv.d:
            raise ValueError("q must be [rows][hq][head_dim] f32")
        o = np.empty((self.rows, hq * kv.d), np.float32)
        check_hip(self.L.yx_attention(self.ctx, kv.h, layer, ptr(q), ptr(o), hq, kv.hkv, w,
                                      scale))
        return o

    # Backend::attention's KV half (lib.rs:132): store the rows' K/V, then attend, in
    # one launch where the plan allows it.
    def attend_append(self, kv, layer, k, v, q, hq, window=None, scale=None, out=None):
        scale = float(np.float32(1.0) / np.sqrt(np.float32(kv.d))) if scale is None else scale
        w = int(window or 0)
        if isinstance(q, DeviceTensor):
            out = out if out is not None else self.tensor((self.rows, hq * kv.d))
            _need(k, self.rows * kv.hkv * kv.d * 4, "k")
            _need(v, self.rows * kv.hkv * kv.d * 4, "v")
            _need(q, self.rows * hq * kv.d * 4, "q")
            _need(out, self.rows * hq * kv.d * 4, "out")
            check_hip(self.L.yx_attention_append_dev(self.ctx, kv.h, layer, k.ptr, v.ptr, q.ptr,
                                                     out.ptr, hq, kv.hkv, w, scale))
            return out
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        if k.size != self.rows * kv.hkv * kv.d or v.size != k.size:
            raise ValueError("k/v must be [rows][hkv][head_dim] f32")
        if q.size != self.rows * hq * kv.d:
            raise ValueError("q must be [rows][hq][head_dim] f32")
        o = np.empty((self.rows, hq * kv.d), np.float32)
        check_hip(self.L.yx_attention_append(self.ctx, kv.h, layer, ptr(k), ptr(v), ptr(q), ptr(o),
                                             hq, kv.hkv, w, scale))
        return o

    def matmul_bf16(self, x, w, out=None):
        """x `[t][k]` f32 device tensor times w `[n][k]` (bf16 bits, uint16 device tensor)
        transposed: `[t][n]` f32 (yx_matmul_bf16_dev)."""
        t, k = x.shape
        n = w.shape[0]
        if w.shape[1] != k:
            raise ValueError("x and w disagree on k")
        out = out if out is not None else self.tensor((t, n))
        _need(out, t * n * 4, "out")
        check_hip(self.L.yx_matmul_bf16_dev(self.ctx, x.ptr, w.ptr, out.ptr, t, k, n))
        return out

    def argmax_rows(self, logits, out=None):
        """The first index of each row's largest value (yx_argmax_rows_dev): a uint32
        device tensor of `rows`."""
        rows, cols = logits.shape
        out = out if out is not None else self.tensor((rows,), np.uint32)
        _need(out, rows * 4, "out")
        check_hip(self.L.yx_argmax_rows_dev(self.ctx, logits.ptr, rows, cols, out.ptr))
        return out

    def stat(self, key):
        """A counter of the context (yx_ctx_get_stat), e.g. "page_entries_sent"."""
        out = ctypes.c_uint64()
        check_hip(self.L.yx_ctx_get_stat(self.ctx, key.encode(), ctypes.byref(out)))
        return out.value

    def checksum(self, dev_ptr, nbytes):
        """XOR of every 8-byte word of a device buffer (yx_dev_checksum)."""
        out = ctypes.c_uint64()
        check_hip(self.L.yx_dev_checksum(self.ctx, dev_ptr, nbytes, ctypes.byref(out)))
        return out.value

    def fill_normal(self, dev_ptr, n, f16, seed, offset=0):
        check_hip(self.L.yx_fill_normal(self.ctx, dev_ptr, n,
                                        _lib.YX_DTYPE_F16 if f16 else _lib.YX_DTYPE_F32,
                                        seed, offset))

    def graph_begin(self):
        check_hip(self.L.yx_graph_begin(self.ctx))

    def graph_end(self):
        check_hip(self.L.yx_graph_end(self.ctx))

    def graph_launch(self):
        check_hip(self.L.yx_graph_launch(self.ctx))

    def timer_start(self):
        check_hip(self.L.yx_timer_start(self.ctx))

    def timer_stop(self):
        ms = ctypes.c_float()
        check_hip(self.L.yx_timer_stop(self.ctx, ctypes.byref(ms)))
        return ms.value

    def profile(self, on):
        check_hip(self.L.yx_profile_enable(self.ctx, 1 if on else 0))

    def profile_read(self, kernel):
        t = ctypes.c_double()
        n = ctypes.c_uint64()
        check_hip(self.L.yx_profile_read(self.ctx, kernel, ctypes.byref(t), ctypes.byref(n)))
        return t.value, n.value
