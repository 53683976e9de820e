//! The (Dense, Gpu) kernel of the boxed operator registry
//! (crates/rusticide-dispatch/src/dispatcher.rs:38-76; key slot from
//! crates/rusticide-core/src/key/kernel_table.rs:105-131).
//!
//! Operator `quantized_matmul`, stack bottom to top:
//! `[Tensor inputs (F32, [tokens, width]) on gpu:i, Int matrix id]` ->
//! `[Tensor out (F32, [rows, tokens]) on gpu:i]`, `out[row][token]` as
//! `matmul_batch` lays it out (matmul.rs:222-229).
//!
//! A `DeviceMatrix` cannot ride on the stack (`IValue` has no opaque
//! handle), so callers register their matrices with a [`Registry`] and pass
//! the id it returns. rusticide-core's storage for a `Device::gpu(i)` tensor
//! is host memory today (crates/rusticide-core/src/storage/mod.rs:40-52), so
//! the kernel reads and writes the tensors' bytes on the host and runs the
//! product through the host-buffer entry point, which stages them through
//! HBM. When rusticide-core gains device storage, the same kernel switches to
//! `matmul_batch_device` on the tensors' device pointers and the context's
//! stream.

use std::collections::HashMap;
use std::sync::atomic::{AtomicI64, Ordering};
use std::sync::{Arc, Mutex, PoisonError};

use rusticide_core::{BackendComponent, DType, DeviceKind, DispatchKey, DispatchKeySet, Tensor};
use rusticide_dispatch::{DispatchError, Dispatcher, IValue, KernelFunction, Stack};

use crate::{Context, DeviceMatrix, matmul_batch};

pub const OPERATOR: &str = "quantized_matmul";

/// The context the kernel runs on and the matrices callers refer to by id.
pub struct Registry {
    ctx: Mutex<Context>,
    matrices: Mutex<HashMap<i64, Arc<DeviceMatrix>>>,
    next: AtomicI64,
}

impl Registry {
    #[must_use]
    pub fn new(ctx: Context) -> Self {
        Self { ctx: Mutex::new(ctx), matrices: Mutex::new(HashMap::new()), next: AtomicI64::new(1) }
    }

    /// Makes `matrix` callable by the returned id.
    pub fn insert(&self, matrix: Arc<DeviceMatrix>) -> i64 {
        let id = self.next.fetch_add(1, Ordering::Relaxed);
        self.matrices.lock().unwrap_or_else(PoisonError::into_inner).insert(id, matrix);
        id
    }

    pub fn remove(&self, id: i64) -> Option<Arc<DeviceMatrix>> {
        self.matrices.lock().unwrap_or_else(PoisonError::into_inner).remove(&id)
    }

    fn get(&self, id: i64) -> Option<Arc<DeviceMatrix>> {
        self.matrices.lock().unwrap_or_else(PoisonError::into_inner).get(&id).cloned()
    }
}

fn failed(reason: impl Into<String>) -> DispatchError {
    DispatchError::KernelFailed(reason.into())
}

/// The f32 values of a byte slice, which the allocator aligns for any
/// element type.
fn as_f32(bytes: &[u8]) -> Result<&[f32], DispatchError> {
    // SAFETY: every bit pattern is a valid f32; align_to only reinterprets
    // the aligned middle part, and the check below refuses any remainder.
    let (head, body, tail) = unsafe { bytes.align_to::<f32>() };
    if head.is_empty() && tail.is_empty() { Ok(body) } else { Err(failed("tensor bytes are not f32-aligned")) }
}

fn as_f32_mut(bytes: &mut [u8]) -> Result<&mut [f32], DispatchError> {
    // SAFETY: as in as_f32; the slice is exclusively borrowed.
    let (head, body, tail) = unsafe { bytes.align_to_mut::<f32>() };
    if head.is_empty() && tail.is_empty() { Ok(body) } else { Err(failed("tensor bytes are not f32-aligned")) }
}

fn run(registry: &Registry, stack: &mut Stack) -> Result<(), DispatchError> {
    let id = stack.pop_int().ok_or_else(|| failed("expected a matrix id on top of the stack"))?;
    let input = stack.pop_tensor().ok_or_else(|| failed("expected an input tensor under the matrix id"))?;
    let matrix = registry.get(id).ok_or_else(|| failed(format!("no matrix registered as {id}")))?;
    if input.device().kind() != DeviceKind::Gpu || input.dtype() != DType::F32 {
        return Err(failed("inputs must be an F32 tensor on a GPU device"));
    }
    let dims = input.shape().dims();
    let (tokens, width) = match *dims {
        [w] => (1, w),
        [t, w] => (t, w),
        _ => return Err(failed("inputs must be [width] or [tokens, width]")),
    };
    if !input.strides().is_contiguous(input.shape()) || input.storage().numel() != tokens * width {
        return Err(failed("inputs must be a whole contiguous tensor"));
    }
    let rows = matrix.rows();
    let out = Tensor::zeros(&[rows, tokens], DType::F32, input.device())?;
    {
        let x = input.storage().read();
        let mut y = out.storage().write();
        let mut ctx = registry.ctx.lock().unwrap_or_else(PoisonError::into_inner);
        let mut jobs = [(matrix.as_ref(), as_f32_mut(&mut y)?)];
        matmul_batch(&mut ctx, as_f32(&x)?, tokens, &mut jobs).map_err(|e| failed(e.to_string()))?;
    }
    out.bump_version();
    stack.push(IValue::Tensor(out));
    Ok(())
}

/// Installs `quantized_matmul` for dense GPU tensors on `dispatcher`.
pub fn register(dispatcher: &Dispatcher, registry: Arc<Registry>) {
    let keys = DispatchKeySet::empty().with_backend(BackendComponent::Gpu).with_functionality(DispatchKey::Dense);
    dispatcher.register(OPERATOR, keys, KernelFunction::new(move |stack: &mut Stack| run(&registry, stack)));
}
