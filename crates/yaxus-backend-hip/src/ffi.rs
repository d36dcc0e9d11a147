//! The C ABI of `include/yaxus_hip.h` (libyaxus_hip.so), declared for Rust. One
//! declaration per function of the header, in its order, with the same argument types:
//! `size_t` is `usize`, `int` is `c_int`, `long` is `c_long`, `float` is `f32`, the two
//! handle types are opaque. `tests/test_rust_ffi.py` in the yaxus_amd repository parses
//! this block and the header and checks that they agree.
//!
//! Conventions (the header's): every call returns a status, `YX_OK` = 0; the message of
//! the last failure on this thread is `yx_last_error()`; all device work of a context
//! goes on its one stream, in call order; the `_dev` variants take device pointers and
//! return before the work is done (`yx_sync` waits).

#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_long, c_void};

/// A device context: one GPU, one stream, the current pass and the attention's scratch.
#[repr(C)]
pub struct yx_ctx {
    _private: [u8; 0],
}

/// The paged K/V arena of one model (every layer).
#[repr(C)]
pub struct yx_kv {
    _private: [u8; 0],
}

pub const YX_OK: c_int = 0;
pub const YX_ERR_INVALID: c_int = 1;
pub const YX_ERR_HIP: c_int = 5;
pub const YX_ERR_UNSUPPORTED: c_int = 6;
pub const YX_DTYPE_F32: c_int = 0;
pub const YX_DTYPE_F16: c_int = 1;
pub const YX_K: c_int = 0;
pub const YX_V: c_int = 1;
pub const YX_KERNEL_ATTENTION: c_int = 0;
pub const YX_KERNEL_APPEND: c_int = 1;
pub const YX_KERNEL_COPY: c_int = 2;
pub const YX_KERNEL_QK_ROPE: c_int = 3;

unsafe extern "C" {
    pub fn yx_last_error() -> *const c_char;
    pub fn yx_device_count(n: *mut c_int) -> c_int;

    pub fn yx_ctx_create(device: c_int, out: *mut *mut yx_ctx) -> c_int;
    pub fn yx_ctx_destroy(ctx: *mut yx_ctx) -> c_int;
    pub fn yx_sync(ctx: *mut yx_ctx) -> c_int;
    pub fn yx_ctx_set_option(ctx: *mut yx_ctx, key: *const c_char, value: c_long) -> c_int;
    pub fn yx_ctx_get_stat(ctx: *mut yx_ctx, key: *const c_char, out: *mut u64) -> c_int;

    pub fn yx_kv_create(ctx: *mut yx_ctx, layers: usize, pages: usize, page_size: usize, hkv: usize,
                        head_dim: usize, dtype: c_int, out: *mut *mut yx_kv) -> c_int;
    pub fn yx_kv_destroy(ctx: *mut yx_ctx, kv: *mut yx_kv) -> c_int;
    pub fn yx_kv_layer_ptr(kv: *mut yx_kv, layer: usize, which: c_int, out: *mut *mut c_void) -> c_int;
    pub fn yx_kv_page_bytes(kv: *const yx_kv) -> usize;

    pub fn yx_kv_copy_pages(ctx: *mut yx_ctx, kv: *mut yx_kv, src: *const u32, dst: *const u32,
                            n: usize) -> c_int;
    pub fn yx_kv_read_pages(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, pages: *const u32,
                            n: usize, k_out: *mut c_void, v_out: *mut c_void) -> c_int;
    pub fn yx_kv_write_pages(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, pages: *const u32,
                             n: usize, k_in: *const c_void, v_in: *const c_void) -> c_int;

    pub fn yx_pass_begin(ctx: *mut yx_ctx, rows: usize, pos: *const u32, kv_slot: *const u32,
                         pt_off: *const u32, pages: *const u32, npages: usize) -> c_int;

    pub fn yx_kv_append(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, k: *const f32,
                        v: *const f32) -> c_int;
    pub fn yx_kv_append_dev(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, k: *const f32,
                            v: *const f32) -> c_int;

    pub fn yx_qk_rope_append_dev(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, qkv: *const f32,
                                 q_norm: *const f32, k_norm: *const f32, rope_cs: *const f32,
                                 rope_len: usize, eps: f32, hq: usize, hkv: usize,
                                 q_out: *mut f32) -> c_int;
    pub fn yx_attention_qkv_dev(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, qkv: *const f32,
                                q_norm: *const f32, k_norm: *const f32, rope_cs: *const f32,
                                rope_len: usize, eps: f32, out: *mut f32, hq: usize, hkv: usize,
                                window: usize, scale: f32) -> c_int;

    pub fn yx_attention(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, q: *const f32, out: *mut f32,
                        hq: usize, hkv: usize, window: usize, scale: f32) -> c_int;
    pub fn yx_attention_dev(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, q: *const f32,
                            out: *mut f32, hq: usize, hkv: usize, window: usize, scale: f32) -> c_int;
    pub fn yx_attention_append(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, k: *const f32,
                               v: *const f32, q: *const f32, out: *mut f32, hq: usize, hkv: usize,
                               window: usize, scale: f32) -> c_int;
    pub fn yx_attention_append_dev(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize, k: *const f32,
                                   v: *const f32, q: *const f32, out: *mut f32, hq: usize,
                                   hkv: usize, window: usize, scale: f32) -> c_int;
    pub fn yx_attention_append_noalloc(ctx: *mut yx_ctx, kv: *mut yx_kv, layer: usize,
                                       k: *const f32, v: *const f32, q: *const f32, out: *mut f32,
                                       hq: usize, hkv: usize, window: usize, scale: f32) -> c_int;

    pub fn yx_matmul_bf16_dev(ctx: *mut yx_ctx, x: *const f32, w: *const u16, out: *mut f32, t: usize,
                              k: usize, n: usize) -> c_int;
    pub fn yx_argmax_rows_dev(ctx: *mut yx_ctx, logits: *const f32, rows: usize, cols: usize,
                              out: *mut u32) -> c_int;

    pub fn yx_dev_alloc(ctx: *mut yx_ctx, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn yx_dev_free(ctx: *mut yx_ctx, p: *mut c_void) -> c_int;
    pub fn yx_host_alloc(ctx: *mut yx_ctx, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn yx_host_free(ctx: *mut yx_ctx, p: *mut c_void) -> c_int;
    pub fn yx_memcpy_h2d(ctx: *mut yx_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn yx_memcpy_d2h(ctx: *mut yx_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn yx_dev_copy(ctx: *mut yx_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn yx_dev_checksum(ctx: *mut yx_ctx, src: *const c_void, bytes: usize, out: *mut u64) -> c_int;
    pub fn yx_fill_normal(ctx: *mut yx_ctx, dst: *mut c_void, n: usize, dtype: c_int, seed: u64,
                          offset: u64) -> c_int;

    pub fn yx_graph_begin(ctx: *mut yx_ctx) -> c_int;
    pub fn yx_graph_end(ctx: *mut yx_ctx) -> c_int;
    pub fn yx_graph_launch(ctx: *mut yx_ctx) -> c_int;

    pub fn yx_timer_start(ctx: *mut yx_ctx) -> c_int;
    pub fn yx_timer_stop(ctx: *mut yx_ctx, ms: *mut f32) -> c_int;
    pub fn yx_profile_enable(ctx: *mut yx_ctx, on: c_int) -> c_int;
    pub fn yx_profile_read(ctx: *mut yx_ctx, kernel: c_int, total_ms: *mut f64,
                           launches: *mut u64) -> c_int;
}

/// `Ok` for `YX_OK`, else the library's message for the failed call.
pub fn check(rc: c_int) -> anyhow::Result<()> {
    if rc == YX_OK {
        return Ok(());
    }
    // SAFETY: yx_last_error returns a NUL-terminated string owned by the library's
    // thread-local state, valid until the next failing call on this thread.
    let msg = unsafe { std::ffi::CStr::from_ptr(yx_last_error()) }.to_string_lossy().into_owned();
    anyhow::bail!("yaxus-hip: {msg} (status {rc})")
}
