//! The `Hip` arm of yaxus-native's backend choice (crates/yaxus-native/src/options.rs:11-27,
//! crates/yaxus-native/src/load.rs:25-64). yaxus-native gains the variant and calls these:
//!
//! - `BackendKind::Hip` ("hip"): [`open`] around the CPU backend (which then implements
//!   [`HostTensors`]); an error when no gfx950 device opens.
//! - `BackendKind::Auto`: [`available`] first; when it holds, the `Hip` arm, else the
//!   existing order (the wgpu/Metal GPU, then the CPU).
//!
//! The device index is `YAXUS_HIP_DEVICE` (default 0): one engine process per GPU.

use anyhow::Result;

use crate::{ffi, HipBackend, HostTensors};

/// The HIP device this process uses.
pub fn device() -> i32 {
    std::env::var("YAXUS_HIP_DEVICE").ok().and_then(|s| s.parse().ok()).unwrap_or(0)
}

/// Whether a gfx950 device opens (a context is created and dropped).
pub fn available() -> bool {
    let mut n = 0;
    // SAFETY: n receives the device count.
    if unsafe { ffi::yx_device_count(&mut n) } != ffi::YX_OK || n <= device() {
        return false;
    }
    let mut ctx = std::ptr::null_mut();
    // SAFETY: a context is created and destroyed at once.
    if unsafe { ffi::yx_ctx_create(device(), &mut ctx) } != ffi::YX_OK {
        return false;
    }
    unsafe { ffi::yx_ctx_destroy(ctx) };
    true
}

/// The HIP backend around `inner` (the CPU backend in yaxus-native).
pub fn open<B: HostTensors>(inner: B) -> Result<HipBackend<B>> {
    HipBackend::new(device(), inner)
}
