//! rusticide-hip: rusticide's quantized matrix products on one MI355X
//! (gfx950), over the C ABI of `librusticide_hip.so`
//! (`include/rusticide_hip.h` in the HIP repository).
//!
//! Like `rusticide-alloc` and `rusticide-simd`, this is a crate permitted
//! `unsafe`: every call into the ABI is an `unsafe` block with its SAFETY
//! argument, and the types here keep the ABI's ownership rules (a context is
//! `Send` but not `Sync`; matrices, quantized inputs and decoders free their
//! device memory on drop).
//!
//! What rusticide binds it to:
//! * `Context::open` is the GPU probe beside `active()`'s CPU adapter choice
//!   (crates/rusticide-kernels/src/adapter.rs:86-169): `None` keeps the CPU
//!   adapter.
//! * `DeviceMatrix::load` is `Matrix::load_on` + `Adapter::prepare_matrix`
//!   for the GPU (crates/rusticide-model/src/weights.rs:53-98,
//!   crates/rusticide-kernels/src/adapter.rs:70-83): the GGUF block bytes
//!   uploaded once.
//! * `matmul_batch` / `matvec_batch` are `matmul_batch` / `matvec_batch`
//!   (crates/rusticide-kernels/src/matmul.rs:218-248) for jobs whose weights
//!   live on the GPU; the outputs are the CPU path's, bit for bit.
//! * `DeviceQ8Input` and `DeviceMatrix::dot_matrix_device` are
//!   `Q8Input::quantize` and `QuantKernel::dot_matrix` /
//!   `dot_ternary_matrix` (q8_input.rs:52-58, quant_kernel.rs:106-119) on
//!   device buffers.
//! * `decoder::HipDecoder` implements the `Model` seam of
//!   crates/rusticide-model/src/generate.rs:35-124 over a device decoder;
//!   `gguf` loads a llama GGUF file straight to HBM.
//! * `dispatch::register` (feature `dispatch`) installs the (Dense, Gpu)
//!   kernel of the boxed operator registry
//!   (crates/rusticide-dispatch/src/dispatcher.rs:38-76).

pub mod decoder;
#[cfg(feature = "dispatch")]
pub mod dispatch;
pub mod gguf;
pub mod sys;

use core::ffi::{CStr, c_int, c_void};
use core::fmt;

/// A failed call: the ABI's status and the library's message for it.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct HipError {
    pub status: sys::rh_status,
    pub message: String,
}

impl fmt::Display for HipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "{:?}: {}", self.status, self.message)
    }
}

impl std::error::Error for HipError {}

pub type Result<T> = std::result::Result<T, HipError>;

fn message(ctx: *const sys::rh_ctx) -> String {
    // SAFETY: rh_last_error accepts any context pointer the library handed
    // out, or null, and returns a NUL-terminated string that lives until the
    // next failing call on that context (or this thread); it is copied here.
    let p = unsafe { sys::rh_last_error(ctx) };
    if p.is_null() {
        return String::new();
    }
    // SAFETY: p is non-null and NUL-terminated (see above).
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

fn check(ctx: *const sys::rh_ctx, status: sys::rh_status) -> Result<()> {
    if status == sys::rh_status::Ok {
        Ok(())
    } else {
        Err(HipError { status, message: message(ctx) })
    }
}

/// `Q8Kind` (crates/rusticide-kernels/src/q8_input.rs:33-50) for the two
/// schemes the device kernels read.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Q8Kind {
    /// Q8_K, paired with Q4_K and Q6_K.
    SuperBlock,
    /// I8_S, paired with I2_S.
    Row,
}

impl Q8Kind {
    const fn raw(self) -> c_int {
        match self {
            Self::SuperBlock => sys::RH_Q8_SUPER_BLOCK,
            Self::Row => sys::RH_Q8_ROW,
        }
    }
}

/// The adapter name, as `Adapter::name` (adapter.rs:40-45): "hip-gfx950".
#[must_use]
pub fn adapter_name() -> &'static str {
    // SAFETY: rh_adapter_name returns a static NUL-terminated string.
    unsafe { CStr::from_ptr(sys::rh_adapter_name()) }.to_str().unwrap_or("hip-gfx950")
}

/// One device and the HIP stream every call on it is queued on. Calls on
/// one context must not overlap, so it is `Send` but not `Sync`.
pub struct Context {
    raw: *mut sys::rh_ctx,
}

// SAFETY: the library keeps no thread-affine state in a context; it only
// requires that calls on one context do not overlap, which `&mut self` and
// the absence of `Sync` guarantee.
unsafe impl Send for Context {}

impl Context {
    /// Opens `device` when it is a gfx950; `None` (no device, another
    /// architecture) tells the caller to keep the CPU adapter.
    #[must_use]
    pub fn open(device: i32) -> Option<Self> {
        let mut raw = core::ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer; on success the library
        // returns an owned context, freed in Drop.
        let status = unsafe { sys::rh_init(device, &raw mut raw) };
        (status == sys::rh_status::Ok && !raw.is_null()).then_some(Self { raw })
    }

    /// The HIP stream (a `hipStream_t`) the context queues work on.
    #[must_use]
    pub fn stream(&mut self) -> *mut c_void {
        // SAFETY: self.raw is a live context.
        unsafe { sys::rh_stream(self.raw) }
    }

    /// The message of the last failed call on this context.
    #[must_use]
    pub fn last_error(&self) -> String {
        message(self.raw)
    }

    pub(crate) const fn raw(&self) -> *mut sys::rh_ctx {
        self.raw
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        // SAFETY: self.raw came from rh_init and is freed once, here. The
        // library drains the context's stream first.
        unsafe { sys::rh_destroy(self.raw) };
    }
}

/// The dense and block formats `Matrix::load` accepts
/// (crates/rusticide-model/src/weights.rs:241-247): GGML type ids.
pub mod types {
    pub const F32: u32 = super::sys::RH_TYPE_F32;
    pub const F16: u32 = super::sys::RH_TYPE_F16;
    pub const Q4_K: u32 = super::sys::RH_TYPE_Q4_K;
    pub const Q6_K: u32 = super::sys::RH_TYPE_Q6_K;
    pub const I2_S: u32 = super::sys::RH_TYPE_I2_S;
}

/// A weight matrix resident in HBM in its GGUF block layout.
pub struct DeviceMatrix {
    raw: *mut sys::rh_matrix,
}

// SAFETY: a loaded matrix is immutable device memory; the library reads it
// from any context on its device, and frees it after draining the device.
unsafe impl Send for DeviceMatrix {}
// SAFETY: as above; no call mutates a matrix.
unsafe impl Sync for DeviceMatrix {}

impl DeviceMatrix {
    /// `Matrix::load_on` for the GPU: `bytes` exactly as
    /// `GgufFile::quantized_tensor` returns them (the I2_S trailer
    /// included), checked as the reference checks them: `MissingKernel`,
    /// `InvalidTensor` (an I2_S scale that is not finite), `ShapeMismatch`,
    /// `InvalidConfig`.
    ///
    /// # Errors
    /// The ABI's status for a refused matrix or a device failure.
    pub fn load(ctx: &mut Context, type_id: u32, bytes: &[u8], rows: usize, cols: usize) -> Result<Self> {
        let mut raw = core::ptr::null_mut();
        // SAFETY: `bytes` is a live slice of `bytes.len()` bytes, copied to
        // the device before the call returns; `raw` is a valid out-pointer.
        let status = unsafe {
            sys::rh_matrix_load(ctx.raw, type_id, bytes.as_ptr().cast(), bytes.len(), rows, cols, &raw mut raw)
        };
        check(ctx.raw, status)?;
        Ok(Self { raw })
    }

    #[must_use]
    pub fn rows(&self) -> usize {
        // SAFETY: self.raw is a live matrix.
        unsafe { sys::rh_matrix_rows(self.raw) }
    }

    #[must_use]
    pub fn cols(&self) -> usize {
        // SAFETY: self.raw is a live matrix.
        unsafe { sys::rh_matrix_cols(self.raw) }
    }

    #[must_use]
    pub fn type_id(&self) -> u32 {
        // SAFETY: self.raw is a live matrix.
        unsafe { sys::rh_matrix_type(self.raw) }
    }

    /// `Weights::Ternary::scale` of an I2_S matrix (0 for other formats).
    #[must_use]
    pub fn ternary_scale(&self) -> f32 {
        // SAFETY: self.raw is a live matrix.
        unsafe { sys::rh_matrix_ternary_scale(self.raw) }
    }

    /// HBM the matrix holds.
    #[must_use]
    pub fn device_bytes(&self) -> usize {
        // SAFETY: self.raw is a live matrix.
        unsafe { sys::rh_matrix_device_bytes(self.raw) }
    }

    /// `Matrix::copy_row` (weights.rs:120-150): row `index` dequantized into
    /// `out`; `Ok(false)` when the row does not exist.
    ///
    /// # Errors
    /// `InvalidArgument` when a dense row does not fit `out`; device failures.
    pub fn copy_row(&self, ctx: &mut Context, index: usize, out: &mut [f32]) -> Result<bool> {
        let mut found: c_int = 0;
        // SAFETY: `out` is a live, writable slice of `out.len()` values, and
        // the call writes at most that many before returning.
        let status =
            unsafe { sys::rh_matrix_copy_row(ctx.raw, self.raw, index, out.as_mut_ptr(), out.len(), &raw mut found) };
        check(ctx.raw, status)?;
        Ok(found != 0)
    }

    /// `QuantKernel::dot_matrix` on device buffers: every row against every
    /// token of `q` into `out[row * tokens + token]` (`out_len` values at
    /// most), queued on `stream` (null: the context's stream).
    ///
    /// # Safety
    /// `out` must be device memory of at least `out_len` floats on the
    /// context's device, live until the queued work ends, and `q` must hold
    /// the kind this matrix pairs with.
    ///
    /// # Errors
    /// `InvalidArgument` for a mismatched kind; launch failures.
    pub unsafe fn dot_matrix_device(
        &self,
        ctx: &mut Context,
        q: &DeviceQ8Input,
        out: *mut f32,
        out_len: usize,
        stream: *mut c_void,
    ) -> Result<()> {
        // SAFETY: the caller guarantees `out`; `q.raw` and `self.raw` are live.
        let status = unsafe { sys::rh_dot_matrix_device(ctx.raw, self.raw, q.raw, out, out_len, stream) };
        check(ctx.raw, status)
    }

    pub(crate) const fn raw(&self) -> *const sys::rh_matrix {
        self.raw
    }
}

impl Drop for DeviceMatrix {
    fn drop(&mut self) {
        // SAFETY: self.raw came from rh_matrix_load and is freed once; the
        // library drains the device before it frees the memory.
        unsafe { sys::rh_matrix_free(self.raw) };
    }
}

/// `matmul_batch` (matmul.rs:229-248) for jobs whose weights live on the
/// GPU: `tokens` rows of `inputs.len() / tokens` values against every job,
/// `out[row * tokens + token]`, each output's length bounding its rows. A
/// no-op when `tokens` is 0 or exceeds `inputs.len()`, as in the reference.
///
/// # Errors
/// `InvalidArgument` for a job without a matrix; device failures.
pub fn matmul_batch(
    ctx: &mut Context,
    inputs: &[f32],
    tokens: usize,
    jobs: &mut [(&DeviceMatrix, &mut [f32])],
) -> Result<()> {
    let raw: Vec<sys::rh_job> = jobs
        .iter_mut()
        .map(|(m, out)| sys::rh_job { weights: m.raw(), out: out.as_mut_ptr(), out_len: out.len() })
        .collect();
    // SAFETY: every job's output is a live, writable host slice of out_len
    // values, `inputs` a live slice; the call is synchronous, so neither
    // outlives the borrow.
    let status = unsafe { sys::rh_matmul_batch(ctx.raw, inputs.as_ptr(), inputs.len(), tokens, raw.as_ptr(), raw.len()) };
    check(ctx.raw, status)
}

/// `matvec_batch` (matmul.rs:218-227): one token.
///
/// # Errors
/// As [`matmul_batch`].
pub fn matvec_batch(ctx: &mut Context, input: &[f32], jobs: &mut [(&DeviceMatrix, &mut [f32])]) -> Result<()> {
    let raw: Vec<sys::rh_job> = jobs
        .iter_mut()
        .map(|(m, out)| sys::rh_job { weights: m.raw(), out: out.as_mut_ptr(), out_len: out.len() })
        .collect();
    // SAFETY: as in matmul_batch.
    let status = unsafe { sys::rh_matvec_batch(ctx.raw, input.as_ptr(), input.len(), raw.as_ptr(), raw.len()) };
    check(ctx.raw, status)
}

/// [`matmul_batch`] on device buffers, queued on `stream` (null: the
/// context's stream); returns without waiting.
///
/// # Safety
/// `inputs` must be device memory of `inputs_len` floats and every job's
/// `out` device memory of `out_len` floats, on the context's device, live
/// until the queued work ends; every job's matrix must outlive it too.
///
/// # Errors
/// As [`matmul_batch`].
pub unsafe fn matmul_batch_device(
    ctx: &mut Context,
    inputs: *const f32,
    inputs_len: usize,
    tokens: usize,
    jobs: &[sys::rh_job],
    stream: *mut c_void,
) -> Result<()> {
    // SAFETY: guaranteed by the caller.
    let status = unsafe { sys::rh_matmul_batch_device(ctx.raw, inputs, inputs_len, tokens, jobs.as_ptr(), jobs.len(), stream) };
    check(ctx.raw, status)
}

/// [`matmul_batch_device`] for callers that cannot allocate device memory
/// (code under HIP graph capture, serving loops): the quantized activations
/// go to a fixed array of `sys::RH_NOALLOC_SCRATCH_BYTES` per GPU, batches
/// that need more are refused, and calls that overlap on one GPU race.
///
/// # Safety
/// As [`matmul_batch_device`]; in addition, no other call of this function
/// may overlap it on the same GPU.
///
/// # Errors
/// `InvalidArgument` for a batch beyond the array; as [`matmul_batch`].
pub unsafe fn matmul_batch_device_noalloc(
    ctx: &mut Context,
    inputs: *const f32,
    inputs_len: usize,
    tokens: usize,
    jobs: &[sys::rh_job],
    stream: *mut c_void,
) -> Result<()> {
    // SAFETY: guaranteed by the caller.
    let status = unsafe {
        sys::rh_matmul_batch_device_noalloc(ctx.raw, inputs, inputs_len, tokens, jobs.as_ptr(), jobs.len(), stream)
    };
    check(ctx.raw, status)
}

/// The batch size from which Q4_K, Q6_K and I2_S matrices run on the MFMA
/// GEMMs instead of the GEMV kernels (both give the same bits). No
/// counterpart in the reference, whose row kernels serve every batch size.
#[must_use]
pub fn gemm_min_tokens() -> usize {
    // SAFETY: a process-wide read with no preconditions.
    unsafe { sys::rh_gemm_min_tokens() }
}

pub fn set_gemm_min_tokens(tokens: usize) {
    // SAFETY: a process-wide store with no preconditions.
    unsafe { sys::rh_set_gemm_min_tokens(tokens) };
}

/// `Q8Input` on the device (q8_input.rs:13-23): a batch of quantized
/// activations, one per token, reused across calls.
pub struct DeviceQ8Input {
    raw: *mut sys::rh_q8,
}

// SAFETY: device memory with no thread-affine state; mutation needs `&mut`.
unsafe impl Send for DeviceQ8Input {}

impl DeviceQ8Input {
    /// # Errors
    /// `OutOfMemory`, device failures.
    pub fn new(ctx: &mut Context) -> Result<Self> {
        let mut raw = core::ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer.
        let status = unsafe { sys::rh_q8_new(ctx.raw, &raw mut raw) };
        check(ctx.raw, status)?;
        Ok(Self { raw })
    }

    /// `Q8Input::quantize` (q8_input.rs:52-58) of each of `tokens` rows of
    /// the device buffer `inputs`, queued on `stream`.
    ///
    /// # Safety
    /// `inputs` must be device memory of `inputs_len` floats on the
    /// context's device, live until the queued work ends.
    ///
    /// # Errors
    /// Device failures.
    pub unsafe fn quantize_device(
        &mut self,
        ctx: &mut Context,
        kind: Q8Kind,
        inputs: *const f32,
        inputs_len: usize,
        tokens: usize,
        stream: *mut c_void,
    ) -> Result<()> {
        // SAFETY: guaranteed by the caller; self.raw is live.
        let status =
            unsafe { sys::rh_q8_quantize_device(ctx.raw, self.raw, kind.raw(), inputs, inputs_len, tokens, stream) };
        check(ctx.raw, status)
    }
}

impl Drop for DeviceQ8Input {
    fn drop(&mut self) {
        // SAFETY: self.raw came from rh_q8_new and is freed once.
        unsafe { sys::rh_q8_free(self.raw) };
    }
}
