"""ctypes bindings of the two native libraries (the C ABI of include/*.h).

Both are loaded from this package's directory; a missing library raises at once —
there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))

YX_OK = 0
YX_ERR_INVALID = 1
YX_ERR_FULL = 2
YX_ERR_LIMIT = 3
YX_ERR_UNKNOWN_SEQ = 4
YX_ERR_HIP = 5
YX_ERR_UNSUPPORTED = 6

YX_DTYPE_F32 = 0
YX_DTYPE_F16 = 1
YX_K = 0
YX_V = 1
YX_KERNEL_ATTENTION = 0
YX_KERNEL_APPEND = 1
YX_KERNEL_COPY = 2
YX_KERNEL_QK_ROPE = 3

P = ctypes.c_void_p
S = ctypes.c_size_t
I = ctypes.c_int
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
F = ctypes.c_float

# name -> (restype, argtypes), exactly the declarations of the headers.
KV_SYMBOLS = {
    "yx_cache_last_error": (ctypes.c_char_p, []),
    "yx_cache_create": (I, [S, S, S, P]),
    "yx_cache_destroy": (None, [P]),
    "yx_cache_set_prefix_reuse": (None, [P, I]),
    "yx_cache_new_seq": (U64, [P]),
    "yx_cache_free_seq": (None, [P, U64]),
    "yx_cache_clear_prefix_cache": (None, [P]),
    "yx_cache_begin": (I, [P, P, S, P, P]),
    "yx_cache_finish": (None, [P, U64]),
    "yx_cache_seq_len": (S, [P, U64]),
    "yx_cache_seq_tokens": (S, [P, U64, P, S]),
    "yx_cache_seq_pages": (S, [P, U64, P, S]),
    "yx_cache_free_pages": (S, [P]),
    "yx_cache_total_pages": (S, [P]),
    "yx_cache_max_pos": (S, [P]),
    "yx_cache_page_size": (S, [P]),
    "yx_cache_page_refs": (U32, [P, U32]),
    "yx_cache_truncate": (I, [P, U64, S]),
    "yx_cache_fork": (I, [P, U64, S, P]),
    "yx_cache_append": (I, [P, S, P, P, P]),
    "yx_cache_pass_rows": (S, [P]),
    "yx_cache_pass_npages": (S, [P]),
    "yx_cache_pass_nitems": (S, [P]),
    "yx_cache_pass_get": (None, [P, P, P, P, P, P, P]),
    "yx_cache_pending_copies": (S, [P]),
    "yx_cache_take_copies": (S, [P, P, S]),
}

HIP_SYMBOLS = {
    "yx_last_error": (ctypes.c_char_p, []),
    "yx_device_count": (I, [P]),
    "yx_ctx_create": (I, [I, P]),
    "yx_ctx_destroy": (I, [P]),
    "yx_sync": (I, [P]),
    "yx_ctx_set_option": (I, [P, ctypes.c_char_p, ctypes.c_long]),
    "yx_kv_create": (I, [P, S, S, S, S, S, I, P]),
    "yx_kv_destroy": (I, [P, P]),
    "yx_kv_layer_ptr": (I, [P, S, I, P]),
    "yx_kv_page_bytes": (S, [P]),
    "yx_kv_copy_pages": (I, [P, P, P, P, S]),
    "yx_kv_read_pages": (I, [P, P, S, P, S, P, P]),
    "yx_kv_write_pages": (I, [P, P, S, P, S, P, P]),
    "yx_pass_begin": (I, [P, S, P, P, P, P, S]),
    "yx_kv_append": (I, [P, P, S, P, P]),
    "yx_kv_append_dev": (I, [P, P, S, P, P]),
    "yx_qk_rope_append_dev": (I, [P, P, S, P, P, P, P, S, F, S, S, P]),
    "yx_attention_qkv_dev": (I, [P, P, S, P, P, P, P, S, F, P, S, S, S, F]),
    "yx_attention": (I, [P, P, S, P, P, S, S, S, F]),
    "yx_attention_dev": (I, [P, P, S, P, P, S, S, S, F]),
    "yx_attention_append": (I, [P, P, S, P, P, P, P, S, S, S, F]),
    "yx_attention_append_dev": (I, [P, P, S, P, P, P, P, S, S, S, F]),
    "yx_attention_append_noalloc": (I, [P, P, S, P, P, P, P, S, S, S, F]),
    "yx_dev_alloc": (I, [P, S, P]),
    "yx_dev_free": (I, [P, P]),
    "yx_host_alloc": (I, [P, S, P]),
    "yx_host_free": (I, [P, P]),
    "yx_memcpy_h2d": (I, [P, P, P, S]),
    "yx_memcpy_d2h": (I, [P, P, P, S]),
    "yx_dev_copy": (I, [P, P, P, S]),
    "yx_dev_checksum": (I, [P, P, S, P]),
    "yx_ctx_get_stat": (I, [P, ctypes.c_char_p, P]),
    "yx_matmul_bf16_dev": (I, [P, P, P, P, S, S, S]),
    "yx_argmax_rows_dev": (I, [P, P, S, S, P]),
    "yx_fill_normal": (I, [P, P, S, I, U64, U64]),
    "yx_graph_begin": (I, [P]),
    "yx_graph_end": (I, [P]),
    "yx_graph_launch": (I, [P]),
    "yx_timer_start": (I, [P]),
    "yx_timer_stop": (I, [P, P]),
    "yx_profile_enable": (I, [P, I]),
    "yx_profile_read": (I, [P, I, P, P]),
}

KV_LIB_PATH = os.path.join(HERE, "libyaxus_kv.so")
HIP_LIB_PATH = os.path.join(HERE, "libyaxus_hip.so")

_kv = None
_hip = None


def _load(path, symbols):
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m yaxus_amd.build` "
            "(the package has no non-native path)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in symbols.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def kv_lib():
    global _kv
    if _kv is None:
        _kv = _load(KV_LIB_PATH, KV_SYMBOLS)
    return _kv


def hip_lib():
    global _hip
    if _hip is None:
        _hip = _load(HIP_LIB_PATH, HIP_SYMBOLS)
    return _hip


class YxError(RuntimeError):
    """An error status from the native library (``code`` is the YX_ERR_* value)."""

    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def check_kv(rc):
    if rc != YX_OK:
        raise YxError(rc, kv_lib().yx_cache_last_error().decode())


def check_hip(rc):
    if rc != YX_OK:
        raise YxError(rc, hip_lib().yx_last_error().decode())


def ptr(a):
    """Address of a numpy array's data."""
    return a.ctypes.data_as(ctypes.c_void_p)
