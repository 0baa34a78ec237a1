//! `rtq`: Rust_Trainer's frozen quantised matmul on an MI355X, through librtq.so's C ABI.
//!
//! The trainer's plugin point is `trait FrozenMatmul` (src/frozen.rs:14-25); its GGUF
//! implementation is `RieFrozen` (src/rie.rs:51-129), built by the loader's `fz` closure
//! (src/rie.rs:183).  [`GpuFrozen`] is built from the same packed GGUF bytes and keeps the same
//! contract: `forward` returns a fresh `y = x·Wᵀ`, `backward_input` accumulates `dx += dy·W`,
//! `row` overwrites one dequantised row, `nbytes` is the GGUF size.  Like the reference, misuse
//! panics (its release profile aborts on panic): every non-zero status becomes a panic carrying
//! the library's message.
//!
//! This crate cannot name the trainer's trait (the trainer depends on it, not the other way
//! round); the trainer implements it with one line, [`impl_frozen_matmul!`]:
//!
//! ```ignore
//! // src/rie.rs of the trainer
//! rtq::impl_frozen_matmul!(crate::frozen::FrozenMatmul);
//! let gpu = rtq::GpuCtx::new(0);
//! let fz = |w: &Weight| -> Frozen {
//!     Arc::new(rtq::GpuFrozen::new(gpu.clone(), ggml_type_of(w), w.data(), w.rows, w.cols))
//! };
//! ```

pub mod ffi;

use std::ffi::{CStr, CString};
use std::os::raw::{c_int, c_void};
use std::sync::Arc;

/// Panics with the library's message on a non-zero status (the reference asserts on misuse).
pub fn check(status: ffi::rtq_status, what: &str) {
    if status != ffi::RTQ_OK {
        let msg = unsafe { CStr::from_ptr(ffi::rtq_last_error()) }.to_string_lossy().into_owned();
        panic!("rtq: {what}: status {status}: {msg}");
    }
}

/// One GPU context: the device, its loaded gfx950 code object, a stream and a workspace.  Calls on
/// one context are serialised inside the library, so it may be shared across threads (the
/// reference's forward runs on the engine pool and its backward on rayon, src/rie.rs:90,139-150).
pub struct GpuCtx(*mut ffi::rtq_ctx);
unsafe impl Send for GpuCtx {}
unsafe impl Sync for GpuCtx {}

impl GpuCtx {
    pub fn new(device: i32) -> Arc<GpuCtx> {
        let mut p = std::ptr::null_mut();
        check(unsafe { ffi::rtq_ctx_create(device as c_int, &mut p) }, "rtq_ctx_create");
        Arc::new(GpuCtx(p))
    }
    pub fn raw(&self) -> *mut ffi::rtq_ctx {
        self.0
    }
    /// Pre-sizes the workspace for calls up to these sizes (optional; it grows on demand).
    pub fn reserve(&self, max_t: usize, max_rows: usize, max_cols: usize, max_rank: usize) {
        check(unsafe { ffi::rtq_ctx_reserve(self.0, max_t as i64, max_rows as i64, max_cols as i64, max_rank as i64) },
              "rtq_ctx_reserve");
    }
}
impl Drop for GpuCtx {
    fn drop(&mut self) {
        unsafe { ffi::rtq_ctx_destroy(self.0) }
    }
}

/// A frozen `[out × in]` weight resident on the GPU: the drop-in for `RieFrozen`.
pub struct GpuFrozen {
    ctx: Arc<GpuCtx>,
    w: *mut ffi::rtq_weight,
    rows: usize,
    cols: usize,
}
unsafe impl Send for GpuFrozen {}
unsafe impl Sync for GpuFrozen {}

impl GpuFrozen {
    /// `ggml_type`: the GGUF tensor type (Q4_0 2, Q8_0 8, Q4_K 12, Q6_K 14; the trainer-native
    /// `FrozenWeight::F32` 0 and `FrozenWeight::Q8_0` 264, src/frozen.rs:33-45); `data`: the packed
    /// bytes of `rows` rows of `cols` elements, as `Weight::data()` gives them (src/rie.rs:186).
    pub fn new(ctx: Arc<GpuCtx>, ggml_type: i32, data: &[u8], rows: usize, cols: usize) -> GpuFrozen {
        let mut w = std::ptr::null_mut();
        check(unsafe {
            ffi::rtq_weight_create(ctx.raw(), ggml_type as c_int, data.as_ptr() as *const c_void, data.len(),
                                   rows as i64, cols as i64, &mut w)
        }, "rtq_weight_create");
        GpuFrozen { ctx, w, rows, cols }
    }
    /// A tensor of a GGUF image opened with [`Gguf`], uploaded straight from the image.
    pub fn from_gguf(ctx: Arc<GpuCtx>, g: &Gguf, name: &str) -> GpuFrozen {
        let c = CString::new(name).expect("tensor name");
        let mut w = std::ptr::null_mut();
        check(unsafe { ffi::rtq_weight_from_gguf(ctx.raw(), g.0, c.as_ptr(), &mut w) }, "rtq_weight_from_gguf");
        let (rows, cols) = unsafe { (ffi::rtq_weight_out_dim(w) as usize, ffi::rtq_weight_in_dim(w) as usize) };
        GpuFrozen { ctx, w, rows, cols }
    }
    pub fn raw(&self) -> *const ffi::rtq_weight {
        self.w
    }
    pub fn ctx(&self) -> &Arc<GpuCtx> {
        &self.ctx
    }

    // FrozenMatmul (src/frozen.rs:14-25)
    pub fn out_dim(&self) -> usize {
        self.rows
    }
    pub fn in_dim(&self) -> usize {
        self.cols
    }
    /// `y[t×out] = x[t×in] · Wᵀ` (a fresh vector, as `RieFrozen::forward`)
    pub fn forward(&self, x: &[f32], t: usize) -> Vec<f32> {
        assert_eq!(x.len(), t * self.cols);
        let mut y = vec![0.0f32; t * self.rows];
        check(unsafe { ffi::rtq_frozen_forward(self.ctx.raw(), self.w, x.as_ptr(), t as i64, y.as_mut_ptr()) },
              "rtq_frozen_forward");
        y
    }
    /// `dx[t×in] += dy[t×out] · W`
    pub fn backward_input(&self, dy: &[f32], t: usize, dx: &mut [f32]) {
        assert_eq!(dy.len(), t * self.rows);
        assert_eq!(dx.len(), t * self.cols);
        check(unsafe { ffi::rtq_frozen_backward_input(self.ctx.raw(), self.w, dy.as_ptr(), t as i64, dx.as_mut_ptr()) },
              "rtq_frozen_backward_input");
    }
    /// one dequantised row (ggml's dequantisation, bit for bit)
    pub fn row(&self, r: usize, out: &mut [f32]) {
        assert_eq!(out.len(), self.cols);
        check(unsafe { ffi::rtq_frozen_row(self.ctx.raw(), self.w, r as i64, out.as_mut_ptr()) }, "rtq_frozen_row");
    }
    /// GGUF bytes of the weight
    pub fn nbytes(&self) -> usize {
        unsafe { ffi::rtq_weight_nbytes(self.w) }
    }

    // Linear with its LoRA on the GPU (src/linear.rs:73-121)
    /// `y = x·Wᵀ (+ bias) (+ (α/r)·(x·Aᵀ)·Bᵀ)`, in `Linear::forward`'s order
    pub fn linear_forward(&self, bias: Option<&[f32]>, lora: Option<&LoraView>, x: &[f32], t: usize) -> Vec<f32> {
        assert_eq!(x.len(), t * self.cols);
        if let Some(b) = bias {
            assert_eq!(b.len(), self.rows);
        }
        let view = lora.map(|l| l.raw(self.rows, self.cols));
        let mut y = vec![0.0f32; t * self.rows];
        check(unsafe {
            ffi::rtq_linear_forward(self.ctx.raw(), self.w, bias.map_or(std::ptr::null(), |b| b.as_ptr()),
                                    view.as_ref().map_or(std::ptr::null(), |v| v as *const _), x.as_ptr(), t as i64,
                                    y.as_mut_ptr())
        }, "rtq_linear_forward");
        y
    }
    /// `Linear::backward`: returns a fresh dx; accumulates `ga += gᵀx`, `gb += (s·dy)ᵀh`
    pub fn linear_backward(&self, lora: Option<(&LoraView, &mut [f32], &mut [f32])>, x: &[f32], dy: &[f32],
                           t: usize) -> Vec<f32> {
        assert_eq!(x.len(), t * self.cols);
        assert_eq!(dy.len(), t * self.rows);
        let mut dx = vec![0.0f32; t * self.cols];
        let (view, ga, gb) = match lora {
            Some((l, ga, gb)) => {
                assert_eq!(ga.len(), l.rank * self.cols);
                assert_eq!(gb.len(), self.rows * l.rank);
                (Some(l.raw(self.rows, self.cols)), ga.as_mut_ptr(), gb.as_mut_ptr())
            }
            None => (None, std::ptr::null_mut(), std::ptr::null_mut()),
        };
        check(unsafe {
            ffi::rtq_linear_backward(self.ctx.raw(), self.w, view.as_ref().map_or(std::ptr::null(), |v| v as *const _),
                                     x.as_ptr(), dy.as_ptr(), t as i64, dx.as_mut_ptr(), ga, gb)
        }, "rtq_linear_backward");
        dx
    }
}
impl Drop for GpuFrozen {
    fn drop(&mut self) {
        unsafe { ffi::rtq_weight_destroy(self.w) }
    }
}

/// A borrowed view of the trainer's `Lora` (src/linear.rs:8-16): host `Vec<f32>` A [rank x in]
/// and B [out x rank], mutated by AdamW between calls.
pub struct LoraView<'a> {
    pub rank: usize,
    pub alpha: f32,
    pub a: &'a [f32],
    pub b: &'a [f32],
    pub enabled: bool,
}
impl LoraView<'_> {
    fn raw(&self, rows: usize, cols: usize) -> ffi::rtq_lora {
        assert_eq!(self.a.len(), self.rank * cols);
        assert_eq!(self.b.len(), rows * self.rank);
        ffi::rtq_lora { rank: self.rank as i64, alpha: self.alpha, a: self.a.as_ptr(), b: self.b.as_ptr(),
                        enabled: self.enabled as c_int }
    }
}

/// A GGUF v3 image (rie_core::gguf::GgufFile): mapped from a path, or borrowing the caller's bytes.
pub struct Gguf(*mut ffi::rtq_gguf);
unsafe impl Send for Gguf {}
unsafe impl Sync for Gguf {}
impl Gguf {
    pub fn open(path: &str) -> Gguf {
        let c = CString::new(path).expect("path");
        let mut g = std::ptr::null_mut();
        check(unsafe { ffi::rtq_gguf_open(c.as_ptr(), &mut g) }, "rtq_gguf_open");
        Gguf(g)
    }
    pub fn raw(&self) -> *const ffi::rtq_gguf {
        self.0
    }
}
impl Drop for Gguf {
    fn drop(&mut self) {
        unsafe { ffi::rtq_gguf_close(self.0) }
    }
}

/// Implements the trainer's `FrozenMatmul` for [`GpuFrozen`] (invoke once, in the trainer crate,
/// with the trait's path).
#[macro_export]
macro_rules! impl_frozen_matmul {
    ($tr:path) => {
        impl $tr for $crate::GpuFrozen {
            fn out_dim(&self) -> usize {
                $crate::GpuFrozen::out_dim(self)
            }
            fn in_dim(&self) -> usize {
                $crate::GpuFrozen::in_dim(self)
            }
            fn forward(&self, x: &[f32], t: usize) -> Vec<f32> {
                $crate::GpuFrozen::forward(self, x, t)
            }
            fn backward_input(&self, dy: &[f32], t: usize, dx: &mut [f32]) {
                $crate::GpuFrozen::backward_input(self, dy, t, dx)
            }
            fn row(&self, r: usize, out: &mut [f32]) {
                $crate::GpuFrozen::row(self, r, out)
            }
            fn nbytes(&self) -> usize {
                $crate::GpuFrozen::nbytes(self)
            }
        }
    };
}
