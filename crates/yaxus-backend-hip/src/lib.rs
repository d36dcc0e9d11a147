//! The KV half of `yaxus_model::Backend` (crates/yaxus-model/src/lib.rs:95-171) on an
//! MI355X: `new_kv`, `copy_page`, `begin_pass` and `attention` run on the HIP kernels of
//! libyaxus_hip.so (the paged arena, page copies, pass metadata, q/k RMSNorm + RoPE +
//! K/V store, and paged decode / verify / prefill attention); every other method of the
//! trait is forwarded to a wrapped backend `B`, which keeps the weights and the
//! activations. Its tensors cross to the device and back at `attention` through
//! [`HostTensors`].
//!
//! Selection: `BackendKind::Hip` in yaxus-native (crates/yaxus-native/src/options.rs:11-27,
//! load.rs:52-64) opens [`HipBackend::new`] around the CPU backend; see [`select`].

pub mod ffi;
pub mod select;

use std::collections::HashMap;
use std::ffi::c_void;
use std::ptr;

use anyhow::Result;
use yaxus_model::{Backend, Config, LayerMeta, PassMeta, Quant, SyncReadback, TensorRef};

use ffi::check;

/// What attention needs from the wrapped backend's values: its activations as host f32
/// rows (`SyncReadback::to_host` and this constructor) and a weight vector's f32 values.
/// The CPU backend implements it in three lines (its `Tensor` is a `Vec<f32>` with a
/// shape; its vectors decode with `Weight::vector_f32`).
pub trait HostTensors: SyncReadback {
    fn tensor_from_host(&mut self, rows: usize, cols: usize, data: Vec<f32>) -> Self::Tensor;
    fn weight_to_host(&self, w: &Self::Weight) -> Vec<f32>;
}

/// Device memory of the context, freed on drop.
struct DevBuf {
    ctx: *mut ffi::yx_ctx,
    ptr: *mut c_void,
    bytes: usize,
}

impl DevBuf {
    fn new(ctx: *mut ffi::yx_ctx, bytes: usize) -> Result<Self> {
        let mut p = ptr::null_mut();
        // SAFETY: ctx is a live context; p receives a device allocation of `bytes`.
        check(unsafe { ffi::yx_dev_alloc(ctx, bytes.max(16), &mut p) })?;
        Ok(DevBuf { ctx, ptr: p, bytes: bytes.max(16) })
    }

    fn upload(ctx: *mut ffi::yx_ctx, data: &[f32]) -> Result<Self> {
        let b = DevBuf::new(ctx, std::mem::size_of_val(data))?;
        // SAFETY: b holds at least size_of_val(data) bytes; the copy is synchronous.
        check(unsafe {
            ffi::yx_memcpy_h2d(ctx, b.ptr, data.as_ptr().cast(), std::mem::size_of_val(data))
        })?;
        Ok(b)
    }

    /// A buffer of at least `bytes`, reallocated only when it must grow.
    fn ensure(slot: &mut Option<DevBuf>, ctx: *mut ffi::yx_ctx, bytes: usize) -> Result<*mut c_void> {
        if slot.as_ref().map_or(true, |b| b.bytes < bytes) {
            *slot = None;
            *slot = Some(DevBuf::new(ctx, bytes.max(1 << 16))?);
        }
        Ok(slot.as_ref().unwrap().ptr)
    }
}

impl Drop for DevBuf {
    fn drop(&mut self) {
        // SAFETY: ptr came from yx_dev_alloc on this context (which waits for the stream).
        unsafe { ffi::yx_dev_free(self.ctx, self.ptr) };
    }
}

/// Pinned (page-locked) host staging for the per-layer copies of a wrapped host
/// backend's tensors: DMA speed both ways, where a pageable Vec is staged through a
/// driver buffer first.
struct PinnedBuf {
    ctx: *mut ffi::yx_ctx,
    ptr: *mut c_void,
    bytes: usize,
}

impl PinnedBuf {
    fn ensure(slot: &mut Option<PinnedBuf>, ctx: *mut ffi::yx_ctx, bytes: usize) -> Result<*mut c_void> {
        if slot.as_ref().map_or(true, |b| b.bytes < bytes) {
            *slot = None;
            let n = bytes.max(1 << 16);
            let mut p = ptr::null_mut();
            // SAFETY: ctx is a live context; p receives n bytes of pinned host memory.
            check(unsafe { ffi::yx_host_alloc(ctx, n, &mut p) })?;
            *slot = Some(PinnedBuf { ctx, ptr: p, bytes: n });
        }
        Ok(slot.as_ref().unwrap().ptr)
    }
}

impl Drop for PinnedBuf {
    fn drop(&mut self) {
        // SAFETY: ptr came from yx_host_alloc on this context (which waits for the stream).
        unsafe { ffi::yx_host_free(self.ctx, self.ptr) };
    }
}

/// The paged K/V arena of one model on the device, with each layer's RoPE table
/// (`[max_pos][head_dim / 2]` cos, then sin, as `Rope::cos_sin` fills it).
pub struct HipKv {
    ctx: *mut ffi::yx_ctx,
    kv: *mut ffi::yx_kv,
    /// Distinct RoPE tables; layers with equal tables share one.
    ropes: Vec<DevBuf>,
    /// Per layer, its table's index in `ropes`.
    rope_of: Vec<usize>,
    max_pos: usize,
}

impl Drop for HipKv {
    fn drop(&mut self) {
        self.ropes.clear();
        // SAFETY: kv was created on ctx, which outlives it (HipBackend owns both).
        unsafe { ffi::yx_kv_destroy(self.ctx, self.kv) };
    }
}

// SAFETY: the handles are used by one engine thread at a time (the engine steps on one
// thread, crates/yaxus-server/src/worker.rs:58-71); the library keeps no thread-bound
// state beyond the error message.
unsafe impl Send for HipKv {}

/// The HIP backend: the KV path on the GPU, the rest on `B`.
pub struct HipBackend<B: HostTensors> {
    inner: B,
    ctx: *mut ffi::yx_ctx,
    rows: usize,
    qkv: Option<DevBuf>,
    out: Option<DevBuf>,
    pin_in: Option<PinnedBuf>,
    pin_out: Option<PinnedBuf>,
    /// Device copies of the q/k norm weights, by the weight's address (cleared with every
    /// new arena: weights live as long as the model that made it).
    norms: HashMap<usize, DevBuf>,
}

// SAFETY: as for HipKv.
unsafe impl<B: HostTensors + Send> Send for HipBackend<B> {}

/// Page size of the arena: the engine's `kv::PAGE` (crates/yaxus-model/src/kv.rs:17).
pub const PAGE: usize = yaxus_model::kv::PAGE;

impl<B: HostTensors> HipBackend<B> {
    /// A context on HIP device `device` (a gfx950 GPU, else an error) around `inner`.
    pub fn new(device: i32, inner: B) -> Result<Self> {
        let mut ctx = ptr::null_mut();
        // SAFETY: ctx receives a new context handle.
        check(unsafe { ffi::yx_ctx_create(device, &mut ctx) })?;
        Ok(HipBackend { inner, ctx, rows: 0, qkv: None, out: None, pin_in: None, pin_out: None,
                        norms: HashMap::new() })
    }

    pub fn inner(&self) -> &B {
        &self.inner
    }

    fn norm(&mut self, w: &B::Weight) -> Result<*const f32> {
        let key = w as *const B::Weight as usize;
        if !self.norms.contains_key(&key) {
            let v = self.inner.weight_to_host(w);
            self.norms.insert(key, DevBuf::upload(self.ctx, &v)?);
        }
        Ok(self.norms[&key].ptr as *const f32)
    }
}

impl<B: HostTensors> Drop for HipBackend<B> {
    fn drop(&mut self) {
        self.qkv = None;
        self.out = None;
        self.pin_in = None;
        self.pin_out = None;
        self.norms.clear();
        // SAFETY: every device buffer of the context is freed above (arenas hold their
        // own context pointer and must be dropped first, as Model drops its Kv first).
        unsafe { ffi::yx_ctx_destroy(self.ctx) };
    }
}

impl<B: HostTensors> Backend for HipBackend<B> {
    type Tensor = B::Tensor;
    type Weight = B::Weight;
    type Kv = HipKv;

    fn name(&self) -> String {
        format!("hip (gfx950) + {}", self.inner.name())
    }
    fn weight_bytes(&self) -> usize {
        self.inner.weight_bytes()
    }
    fn load_weight(&mut self, t: &TensorRef, quant: Quant) -> Result<Self::Weight> {
        self.inner.load_weight(t, quant)
    }
    fn load_embedding(&mut self, t: &TensorRef) -> Result<Self::Weight> {
        self.inner.load_embedding(t)
    }
    fn reserve_activations(&mut self, cfg: &Config, rows: usize) {
        self.inner.reserve_activations(cfg, rows)
    }

    // lib.rs:118 — binary16 K/V (the f32 arena, YX_DTYPE_F32, keeps the CPU backend's
    // K/V bits at about half the decode rate per key), one RoPE table per layer.
    fn new_kv(&mut self, cfg: &Config, metas: &[LayerMeta], pages: usize, max_pos: usize) -> Result<HipKv> {
        let mut kv = ptr::null_mut();
        // SAFETY: kv receives a new arena of the context.
        check(unsafe {
            ffi::yx_kv_create(self.ctx, metas.len(), pages, PAGE, cfg.num_key_value_heads,
                              cfg.head_dim, ffi::YX_DTYPE_F16, &mut kv)
        })?;
        let mut arena = HipKv { ctx: self.ctx, kv, ropes: Vec::new(), rope_of: Vec::new(), max_pos };
        self.norms.clear();
        let half = cfg.head_dim / 2;
        // Tables already on the device, with their host copies: a layer whose table
        // equals one of them (bit for bit) shares it (full and sliding layers usually
        // differ only in the rope base, so a model holds one or two).
        let mut seen: Vec<Vec<f32>> = Vec::new();
        for m in metas {
            let mut t = vec![0f32; 2 * max_pos * half];
            let (cos, sin) = t.split_at_mut(max_pos * half);
            for p in 0..max_pos {
                m.rope.cos_sin(p, &mut cos[p * half..(p + 1) * half], &mut sin[p * half..(p + 1) * half]);
            }
            let same = |a: &Vec<f32>| a.iter().zip(&t).all(|(x, y)| x.to_bits() == y.to_bits());
            match seen.iter().position(same) {
                Some(i) => arena.rope_of.push(i),
                None => {
                    arena.ropes.push(DevBuf::upload(self.ctx, &t)?);
                    arena.rope_of.push(seen.len());
                    seen.push(t);
                }
            }
        }
        Ok(arena)
    }

    // lib.rs:120 — one page in every layer, K and V (the ABI takes batches; the engine
    // calls this per PageCopy, kv.rs:35).
    fn copy_page(&mut self, kv: &mut HipKv, src: u32, dst: u32) {
        // SAFETY: one-element page lists on the stack, valid for the call.
        check(unsafe { ffi::yx_kv_copy_pages(self.ctx, kv.kv, &src, &dst, 1) }).expect("copy_page");
    }

    // lib.rs:123 — the wrapped backend needs the token ids (embed); the device the rows'
    // positions, slots and page tables.
    fn begin_pass(&mut self, pass: &PassMeta) {
        self.inner.begin_pass(pass);
        // SAFETY: the slices outlive the call, which copies them.
        check(unsafe {
            ffi::yx_pass_begin(self.ctx, pass.pos.len(), pass.pos.as_ptr(), pass.kv_slot.as_ptr(),
                               pass.pt_off.as_ptr(), pass.pages.as_ptr(), pass.pages.len())
        })
        .expect("begin_pass");
        self.rows = pass.pos.len();
    }

    fn embed(&mut self, table: &Self::Weight) -> Self::Tensor {
        self.inner.embed(table)
    }
    fn rmsnorm(&mut self, x: &Self::Tensor, w: &Self::Weight, offset: f32, eps: f32) -> Self::Tensor {
        self.inner.rmsnorm(x, w, offset, eps)
    }
    fn matmul(&mut self, x: &Self::Tensor, w: &Self::Weight) -> Self::Tensor {
        self.inner.matmul(x, w)
    }

    // lib.rs:132 — write_rows then attend (backend-cpu lib.rs:516-530): one
    // yx_attention_qkv_dev call (one launch for decode passes).
    fn attention(&mut self, qkv: &Self::Tensor, q_norm: &Self::Weight, k_norm: &Self::Weight,
                 kv: &mut HipKv, cfg: &Config, layer: &LayerMeta) -> Self::Tensor {
        let rows = self.rows;
        let (hq, hkv, d) = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim);
        let host = self.inner.to_host(qkv);
        assert_eq!(host.len(), rows * (hq + 2 * hkv) * d, "attention rows differ from the pass");
        let qn = self.norm(q_norm).expect("q_norm upload");
        let kn = self.norm(k_norm).expect("k_norm upload");
        let bytes_in = std::mem::size_of_val(host.as_slice());
        let bytes_out = rows * hq * d * 4;
        let dq = DevBuf::ensure(&mut self.qkv, self.ctx, bytes_in).expect("device buffer");
        let dout = DevBuf::ensure(&mut self.out, self.ctx, bytes_out).expect("device buffer");
        let pin_in = PinnedBuf::ensure(&mut self.pin_in, self.ctx, bytes_in).expect("pinned buffer");
        let pin_out = PinnedBuf::ensure(&mut self.pin_out, self.ctx, bytes_out).expect("pinned buffer");
        let mut out = vec![0f32; rows * hq * d];
        let scale = 1.0 / (d as f32).sqrt();
        let rope = kv.ropes[kv.rope_of[layer.index]].ptr as *const f32;
        // SAFETY: device and pinned buffers sized above; the device copies are synchronous,
        // so the pinned buffers are free again when each returns.
        unsafe {
            ptr::copy_nonoverlapping(host.as_ptr().cast::<u8>(), pin_in.cast::<u8>(), bytes_in);
            check(ffi::yx_memcpy_h2d(self.ctx, dq, pin_in, bytes_in)).expect("upload");
            check(ffi::yx_attention_qkv_dev(self.ctx, kv.kv, layer.index, dq as *const f32, qn, kn,
                                            rope, kv.max_pos, cfg.rms_norm_eps, dout as *mut f32, hq,
                                            hkv, layer.window.unwrap_or(0), scale))
                .expect("attention");
            check(ffi::yx_memcpy_d2h(self.ctx, pin_out, dout, bytes_out)).expect("download");
            ptr::copy_nonoverlapping(pin_out.cast::<u8>(), out.as_mut_ptr().cast::<u8>(), bytes_out);
        }
        self.inner.tensor_from_host(rows, hq * d, out)
    }

    fn swiglu(&mut self, x: &Self::Tensor) -> Self::Tensor {
        self.inner.swiglu(x)
    }
    fn add_assign(&mut self, a: &mut Self::Tensor, b: &Self::Tensor) {
        self.inner.add_assign(a, b)
    }
    #[allow(clippy::too_many_arguments)]
    fn add_norm(&mut self, x: &mut Self::Tensor, delta: &Self::Tensor, post_w: &Self::Weight,
                post_offset: f32, pre_w: &Self::Weight, pre_offset: f32, eps: f32) -> Self::Tensor {
        self.inner.add_norm(x, delta, post_w, post_offset, pre_w, pre_offset, eps)
    }
    fn matmul_glu(&mut self, x: &Self::Tensor, w: &Self::Weight) -> Self::Tensor {
        self.inner.matmul_glu(x, w)
    }
    fn select_rows(&mut self, x: &Self::Tensor, rows: &[usize]) -> Self::Tensor {
        self.inner.select_rows(x, rows)
    }
}

impl<B: HostTensors> SyncReadback for HipBackend<B> {
    fn argmax_rows(&mut self, logits: &Self::Tensor) -> Vec<u32> {
        self.inner.argmax_rows(logits)
    }
    fn to_host(&mut self, x: &Self::Tensor) -> Vec<f32> {
        self.inner.to_host(x)
    }
}
