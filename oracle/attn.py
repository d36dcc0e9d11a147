"""ctypes wrapper of ``oracle/libattn_oracle.so`` (test infrastructure only).

The C file restates yaxus-backend-cpu's path arithmetic; see the citations there.
Arena layout is the reference CPU backend's: slot-major ``[slots][hkv * d]``.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libattn_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `make -C oracle`")
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        S = ctypes.c_size_t
        L.orc_f32_to_f16_n.argtypes = [P, P, S]
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_store_kv.argtypes = [P, P, ctypes.c_int, S, S, P, P, P]
        L.orc_write_rows.argtypes = [P, S, S, S, S, P, P, ctypes.c_float, P, ctypes.c_float,
                                     P, P, P, P, ctypes.c_int, P]
        L.orc_copy_page.argtypes = [P, P, ctypes.c_int, S, S, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_attend.argtypes = [P, S, S, S, S, P, P, P, S, S, P, P, ctypes.c_int, P, ctypes.c_int]
        L.orc_attend_f64.argtypes = [P, S, S, S, S, P, P, P, S, S, P, P, ctypes.c_int, P]
        L.orc_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64, S, P]
        L.orc_cos_sin.argtypes = [P, S, ctypes.c_float, S, P, P]
        L.orc_dot.argtypes = [P, P, S]
        L.orc_dot.restype = ctypes.c_float
        L.orc_matmul_bf16.argtypes = [P, S, S, P, S, P]
        L.orc_argmax.argtypes = [P, S]
        L.orc_argmax.restype = ctypes.c_uint32
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def normal(n, seed, offset=0):
    """N(0,1) f32 inputs (splitmix64 -> Box-Muller, glibc libm): the same bits on every
    host of this image."""
    out = np.empty(int(n), dtype=np.float32)
    lib().orc_normal(seed, offset, int(n), _p(out))
    return out


def cos_sin_table(inv_freq, concentration, n):
    """`[2][n][half]` cos then sin of positions 0..n-1 (config.rs:213-219)."""
    f = np.ascontiguousarray(inv_freq, dtype=np.float32)
    out = np.empty((2, n, f.size), dtype=np.float32)
    for p in range(n):
        lib().orc_cos_sin(_p(f), f.size, concentration, p, _p(out[0, p]), _p(out[1, p]))
    return out


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


class OracleArena:
    """One layer's KV arena of ``pages * page`` slots, slot-major like the CPU backend."""

    def __init__(self, pages, page, hkv, d, f16=True):
        self.pages, self.page, self.hkv, self.d, self.f16 = pages, page, hkv, d, f16
        self.kvd = hkv * d
        dt = np.uint16 if f16 else np.float32
        self.k = np.zeros((pages * page, self.kvd), dtype=dt)
        self.v = np.zeros((pages * page, self.kvd), dtype=dt)

    def store(self, kv_slot, k, v):
        kv_slot = np.ascontiguousarray(kv_slot, dtype=np.uint32)
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(len(kv_slot), self.kvd)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(len(kv_slot), self.kvd)
        if len(kv_slot) and int(kv_slot.max()) >= self.pages * self.page:
            raise ValueError("slot beyond the arena")
        lib().orc_store_kv(_p(self.k), _p(self.v), int(self.f16), self.kvd, len(kv_slot),
                           _p(kv_slot), _p(k), _p(v))

    def write_rows(self, qkv, hq, qn, kn, eps, inv_freq, concentration, pos, kv_slot):
        rows = len(pos)
        qkv = np.ascontiguousarray(qkv, dtype=np.float32)
        qn = np.ascontiguousarray(qn, dtype=np.float32)
        kn = np.ascontiguousarray(kn, dtype=np.float32)
        inv_freq = np.ascontiguousarray(inv_freq, dtype=np.float32)
        pos = np.ascontiguousarray(pos, dtype=np.uint32)
        kv_slot = np.ascontiguousarray(kv_slot, dtype=np.uint32)
        q = np.zeros((rows, hq * self.d), dtype=np.float32)
        lib().orc_write_rows(_p(qkv), rows, hq, self.hkv, self.d, _p(qn), _p(kn), eps,
                             _p(inv_freq), concentration, _p(pos), _p(kv_slot), _p(self.k),
                             _p(self.v), int(self.f16), _p(q))
        return q

    def copy_page(self, src, dst):
        lib().orc_copy_page(_p(self.k), _p(self.v), int(self.f16), self.kvd, self.page, src, dst)

    def attend(self, q, hq, pos, pt_off, pages, window=0, threads=1):
        rows = len(pos)
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(rows, hq * self.d)
        pos = np.ascontiguousarray(pos, dtype=np.uint32)
        pt_off = np.ascontiguousarray(pt_off, dtype=np.uint32)
        pages = np.ascontiguousarray(pages, dtype=np.uint32)
        out = np.zeros((rows, hq * self.d), dtype=np.float32)
        lib().orc_attend(_p(q), rows, hq, self.hkv, self.d, _p(pos), _p(pt_off), _p(pages),
                         self.page, window or 0, _p(self.k), _p(self.v), int(self.f16), _p(out),
                         threads)
        return out

    def attend_f64(self, q, hq, pos, pt_off, pages, window=0):
        rows = len(pos)
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(rows, hq * self.d)
        pos = np.ascontiguousarray(pos, dtype=np.uint32)
        pt_off = np.ascontiguousarray(pt_off, dtype=np.uint32)
        pages = np.ascontiguousarray(pages, dtype=np.uint32)
        out = np.zeros((rows, hq * self.d), dtype=np.float64)
        lib().orc_attend_f64(_p(q), rows, hq, self.hkv, self.d, _p(pos), _p(pt_off), _p(pages),
                             self.page, window or 0, _p(self.k), _p(self.v), int(self.f16),
                             _p(out))
        return out

    def page_bits(self, page):
        """K and V of one page as ``[hkv][page][d]`` (the device layout's order)."""
        s = slice(page * self.page, (page + 1) * self.page)
        k = self.k[s].reshape(self.page, self.hkv, self.d).transpose(1, 0, 2)
        v = self.v[s].reshape(self.page, self.hkv, self.d).transpose(1, 0, 2)
        return np.ascontiguousarray(k), np.ascontiguousarray(v)


def matmul_bf16(x, w_bits):
    """The CPU backend's matmul with a bf16 weight: x `[t][k]` f32, w `[n][k]` bf16 bits
    (uint16) -> `[t][n]` f32 (lib.rs:234-248, 314-345)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    t, k = x.shape
    n = w.shape[0]
    out = np.empty((t, n), dtype=np.float32)
    lib().orc_matmul_bf16(_p(x), t, k, _p(w), n, _p(out))
    return out


def argmax_rows(logits):
    """The CPU backend's argmax of every row (lib.rs:432-440, 556-558)."""
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return np.array([lib().orc_argmax(_p(a[r]), a.shape[1]) for r in range(a.shape[0])], np.uint32)
