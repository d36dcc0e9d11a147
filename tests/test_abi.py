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
