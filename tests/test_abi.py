"""The C ABI: both libraries load (no GPU needed to load) and export every function
`include/*.h` declares; the ctypes tables bind exactly those, with as many arguments."""

import ctypes
import os
import re

import pytest

from yaxus_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(yx_[a-z_0-9]+)\s*\(([^;]*?)\)\s*;",
                  re.M | re.S)


def _decls(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, args in DECL.findall(text):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


@pytest.mark.parametrize("header,table,loader", [
    ("yaxus_kv_cache.h", _lib.KV_SYMBOLS, _lib.kv_lib),
    ("yaxus_hip.h", _lib.HIP_SYMBOLS, _lib.hip_lib),
])
def test_every_declared_symbol_is_exported_and_bound(header, table, loader):
    decls = _decls(header)
    assert len(decls) >= 10
    lib = loader()
    for name, nargs in decls.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in table, f"{name} has no ctypes binding"
        assert len(table[name][1]) == nargs, f"{name}: {len(table[name][1])} bound, {nargs} declared"
    assert set(table) == set(decls)


def test_no_device_calls_on_load_and_errors_without_a_device():
    lib = _lib.hip_lib()
    assert isinstance(lib.yx_last_error(), bytes)
    c = ctypes.c_void_p()
    n = ctypes.c_int(-1)
    rc = lib.yx_device_count(ctypes.byref(n))
    if rc != 0 or n.value == 0:
        # No GPU here: creating a context fails with a status, not a crash.
        assert lib.yx_ctx_create(0, ctypes.byref(c)) != 0
        assert lib.yx_last_error()


def test_allocator_abi_refuses_null_arguments():
    """The host allocator's entry points return a status (or an empty answer) for null
    handles and arrays instead of dereferencing them."""
    lib = _lib.kv_lib()
    ok = 0
    assert lib.yx_cache_create(8, 1024, 16, None) != ok
    assert lib.yx_cache_create(1 << 30, 1024, 1 << 40, ctypes.byref(ctypes.c_void_p())) != ok
    c = ctypes.c_void_p()
    assert lib.yx_cache_create(8, 1024, 16, ctypes.byref(c)) == ok
    try:
        seq = ctypes.c_uint64(0)
        reused = ctypes.c_size_t(0)
        assert lib.yx_cache_begin(None, None, 0, ctypes.byref(seq), ctypes.byref(reused)) != ok
        assert lib.yx_cache_begin(c, None, 3, ctypes.byref(seq), ctypes.byref(reused)) != ok
        assert lib.yx_cache_begin(c, None, 0, None, ctypes.byref(reused)) != ok
        s = lib.yx_cache_new_seq(c)
        ids = (ctypes.c_uint64 * 1)(s)
        counts = (ctypes.c_size_t * 1)(2)
        assert lib.yx_cache_append(c, 1, ids, counts, None) != ok
        assert lib.yx_cache_append(c, 1, None, counts, None) != ok
        assert lib.yx_cache_append(None, 0, None, None, None) != ok
        assert lib.yx_cache_fork(c, s, 0, None) != ok
        assert lib.yx_cache_truncate(None, s, 0) != ok
        assert lib.yx_cache_seq_tokens(c, s, None, 4) == 0
        assert lib.yx_cache_take_copies(c, None, 4) == 0
        assert lib.yx_cache_free_pages(None) == 0
        assert lib.yx_cache_new_seq(None) == 0
        lib.yx_cache_pass_get(None, None, None, None, None, None, None)
        lib.yx_cache_finish(None, s)
        lib.yx_cache_free_seq(None, s)
        # The cache still works.
        toks = (ctypes.c_uint32 * 2)(5, 6)
        assert lib.yx_cache_append(c, 1, ids, counts, toks) == ok
        assert lib.yx_cache_seq_len(c, s) == 2
    finally:
        lib.yx_cache_destroy(c)
