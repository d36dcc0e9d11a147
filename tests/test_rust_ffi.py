"""The Rust FFI crate (crates/yaxus-backend-hip) against the C header it binds.

No Rust toolchain is installed here, so the crate is checked as text: every function
include/yaxus_hip.h declares appears in src/ffi.rs's `extern "C"` block with the same
name, argument count, argument types and return type (C types mapped to their Rust FFI
spelling), and no other; the constants the crate defines equal the header's; and
src/lib.rs implements the four Backend methods of the path (new_kv, copy_page,
begin_pass, attention; crates/yaxus-model/src/lib.rs:118-140) through those calls.
"""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "crates", "yaxus-backend-hip")

# C spelling (whitespace-normalised) -> Rust FFI spelling.
C_TO_RUST = {
    "void": "()",
    "int": "c_int",
    "long": "c_long",
    "float": "f32",
    "size_t": "usize",
    "uint64_t": "u64",
    "const char*": "*const c_char",
    "int*": "*mut c_int",
    "float*": "*mut f32",
    "double*": "*mut f64",
    "const float*": "*const f32",
    "const uint32_t*": "*const u32",
    "uint32_t*": "*mut u32",
    "const uint16_t*": "*const u16",
    "uint64_t*": "*mut u64",
    "void*": "*mut c_void",
    "const void*": "*const c_void",
    "void**": "*mut *mut c_void",
    "yx_ctx*": "*mut yx_ctx",
    "yx_ctx**": "*mut *mut yx_ctx",
    "yx_kv*": "*mut yx_kv",
    "yx_kv**": "*mut *mut yx_kv",
    "const yx_kv*": "*const yx_kv",
}


def _norm_c(t):
    t = " ".join(t.split())
    return re.sub(r"\s*\*", "*", t)


def _c_decls():
    text = open(os.path.join(ROOT, "include", "yaxus_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    pat = re.compile(r"^\s*((?:const\s+)?[a-z_0-9]+\s*\*?)\s*(yx_[a-z_0-9]+)\s*\(([^;]*?)\)\s*;", re.M | re.S)
    for ret, name, args in pat.findall(text):
        args = args.strip()
        types = []
        if args not in ("", "void"):
            for a in args.split(","):
                a = " ".join(a.split())
                m = re.match(r"(.*?)([A-Za-z_][A-Za-z_0-9]*)$", a)
                types.append(_norm_c(m.group(1)))
        out[name] = (_norm_c(ret), types)
    return out


def _rust_decls():
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for name, args, ret in re.findall(r"pub fn (yx_[a-z_0-9]+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        types = []
        for a in [x for x in args.split(",") if x.strip()]:
            types.append(" ".join(a.split(":", 1)[1].split()))
        out[name] = (" ".join(ret.split()) if ret else "()", types)
    return out


def test_every_header_function_is_declared_in_ffi_rs_with_the_same_types():
    c, r = _c_decls(), _rust_decls()
    assert len(c) >= 30
    assert set(c) == set(r), f"only in the header: {set(c) - set(r)}; only in ffi.rs: {set(r) - set(c)}"
    for name, (cret, cargs) in c.items():
        rret, rargs = r[name]
        assert C_TO_RUST[cret] == rret, f"{name}: returns {cret} in C, {rret} in Rust"
        assert len(cargs) == len(rargs), f"{name}: {len(cargs)} C arguments, {len(rargs)} in Rust"
        for i, (ct, rt) in enumerate(zip(cargs, rargs)):
            assert C_TO_RUST[ct] == rt, f"{name} argument {i}: {ct} in C, {rt} in Rust"


def test_constants_match_the_headers():
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    consts = {k: int(v) for k, v in re.findall(r"pub const (YX_[A-Z_0-9]+): c_int = (\d+);", text)}
    header = open(os.path.join(ROOT, "include", "yaxus_hip.h")).read()
    header += open(os.path.join(ROOT, "include", "yaxus_kv_cache.h")).read()
    hvals = {k: int(v) for k, v in re.findall(r"\b(YX_[A-Z_0-9]+)\s*=\s*(\d+)", header)}
    assert len(consts) >= 10
    for k, v in consts.items():
        assert hvals.get(k) == v, f"{k} = {v} in ffi.rs, {hvals.get(k)} in the headers"


def test_lib_rs_implements_the_backend_methods_of_the_path():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    calls = {"new_kv": "yx_kv_create", "copy_page": "yx_kv_copy_pages",
             "begin_pass": "yx_pass_begin", "attention": "yx_attention_qkv_dev"}
    for method, ffi_fn in calls.items():
        m = re.search(r"fn %s\(.*?\n    \}\n" % method, text, re.S)
        assert m, f"Backend::{method} missing"
        assert ffi_fn in m.group(0), f"Backend::{method} does not call {ffi_fn}"
    assert "impl<B: HostTensors> Backend for HipBackend<B>" in text
    assert "impl<B: HostTensors> SyncReadback for HipBackend<B>" in text
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "yaxus-backend-hip"' in cargo and "yaxus-model" in cargo
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=yaxus_hip" in build
