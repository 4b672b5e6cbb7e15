//! MI355X drop-in for the fused per-layer ops of `atlas-ops` / `atlas-metal`.
//!
//! Two surfaces, as in the reference:
//! * [`NeuralOps`]: the host-slice operator API of `atlas_ops::NeuralOps`
//!   (crates/atlas-ops/src/lib.rs:20-147) -- same method names, argument
//!   order and `(Vec<f32>, DispatchTiming)` results, the same `InvalidInput`
//!   predicates (crates/atlas-metal/src/lib.rs:1400-1408, 1444-1458,
//!   1493-1500, 1705-1713).
//! * [`HipRuntime`] + [`DeviceBuffer`]: the resident path the executors use
//!   (`ResidentCommand`, crates/atlas-metal/src/lib.rs:242-756): device
//!   buffers, asynchronous fused ops on the context's stream, `finish` =
//!   [`HipRuntime::finish`].  The ops the Gemma and Llama executors dispatch
//!   by kernel name map to one method each; [`ffi`] has every entry point.
//!
//! Errors follow `MetalError` (crates/atlas-metal/src/lib.rs:37-53).
pub mod ffi;

use std::ffi::{CStr, CString};
use std::fmt;
use std::marker::PhantomData;
use std::os::raw::{c_int, c_void};
use std::time::Duration;

/// `MetalError`'s kinds that the HIP library reports.
#[derive(Debug, Clone, PartialEq, Eq)]
pub enum HipError {
    NoDevice,
    CommandFailed(String),
    InvalidInput(String),
    OutOfMemory(String),
}

impl fmt::Display for HipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            HipError::NoDevice => write!(f, "no HIP device is available"),
            HipError::CommandFailed(m) => write!(f, "HIP command failed: {m}"),
            HipError::InvalidInput(m) => write!(f, "invalid buffer/input: {m}"),
            HipError::OutOfMemory(m) => write!(f, "HIP device out of memory: {m}"),
        }
    }
}

impl std::error::Error for HipError {}

/// `atlas_ops::OperatorError` (crates/atlas-ops/src/lib.rs:15-19).
#[derive(Debug, Clone, PartialEq, Eq)]
pub enum OperatorError {
    Hip(HipError),
}

impl fmt::Display for OperatorError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            OperatorError::Hip(e) => e.fmt(f),
        }
    }
}

impl std::error::Error for OperatorError {}

impl From<HipError> for OperatorError {
    fn from(e: HipError) -> Self {
        OperatorError::Hip(e)
    }
}

/// `DispatchTiming` (crates/atlas-metal/src/lib.rs:81-88): host wall time of
/// the call and the GPU time between events around its launches.
#[derive(Debug, Clone, Copy)]
pub struct DispatchTiming {
    pub wall_time: Duration,
    pub command_buffer_schedule: Duration,
    pub gpu_time: Option<Duration>,
    pub gpu_idle_gap: Option<Duration>,
}

impl From<ffi::AtlasDispatchTiming> for DispatchTiming {
    fn from(t: ffi::AtlasDispatchTiming) -> Self {
        DispatchTiming {
            wall_time: Duration::from_secs_f64(t.wall_ms.max(0.0) / 1e3),
            command_buffer_schedule: Duration::ZERO,
            gpu_time: Some(Duration::from_secs_f64(t.gpu_ms.max(0.0) / 1e3)),
            gpu_idle_gap: None,
        }
    }
}

/// Row-sum order of the normalisations (`atlas_hip_set_reduction`).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Reduction {
    /// Left-to-right f32 fold: bit-identical to the reference CPU operators.
    Sequential,
    /// Lane-parallel partial sums and a cross-lane tree everywhere.
    Wide,
    /// The library default: tree where the output is a plain scaled row,
    /// the sequential fold where an epilogue can cancel.
    Auto,
}

mod sealed {
    pub trait Sealed {}
    impl Sealed for f32 {}
    impl Sealed for u32 {}
    impl Sealed for u16 {}
    impl Sealed for u8 {}
}

/// Element types a [`DeviceBuffer`] may hold: plain data with no padding and
/// no invalid bit patterns, so bytes read back from the device are always a
/// valid value.  Sealed; implemented for `f32`, `u32`, `u16` (binary16 bits)
/// and `u8` (packed GGUF blocks).
pub trait DevicePod: Copy + sealed::Sealed {}
impl DevicePod for f32 {}
impl DevicePod for u32 {}
impl DevicePod for u16 {}
impl DevicePod for u8 {}

fn invalid(msg: String) -> HipError {
    HipError::InvalidInput(msg)
}

/// The product of `factors` as an element count; InvalidInput when it
/// overflows.
fn extent(factors: &[u64]) -> Result<usize, HipError> {
    let mut p: u64 = 1;
    for &f in factors {
        p = p.checked_mul(f).ok_or_else(|| invalid("buffer extent overflows".into()))?;
    }
    usize::try_from(p).map_err(|_| invalid("buffer extent overflows".into()))
}

/// InvalidInput unless `buf` holds at least `count` elements: the safe
/// resident ops check every buffer against the elements the kernel touches
/// before the call, so no argument can make a kernel read or write past a
/// buffer.
fn holds<T: DevicePod>(buf: &DeviceBuffer<T>, count: usize, what: &str) -> Result<(), HipError> {
    if buf.len() < count {
        return Err(invalid(format!("{what} holds {} elements, the op touches {count}", buf.len())));
    }
    Ok(())
}

/// Bytes of one packed row of `hidden` values (the GGUF block sizes,
/// crates/atlas-core/src/gguf.rs:16-77); None for a format the gathers do
/// not take.  The library rejects widths that are not whole blocks.
fn packed_row_bytes(format: u32, hidden: u32) -> Option<u64> {
    let h = hidden as u64;
    match format {
        ffi::ATLAS_GGUF_Q4_0 => Some(h / 32 * 18),
        ffi::ATLAS_GGUF_Q8_0 => Some(h / 32 * 34),
        ffi::ATLAS_GGUF_Q6_K => Some(h / 256 * 210),
        _ => None,
    }
}

/// One HIP device context: `MetalRuntime::new` (crates/atlas-metal/src/lib.rs:909-1061).
/// Use it from one thread at a time (calls are not re-entrant).
pub struct HipRuntime {
    ctx: *mut ffi::AtlasHipCtx,
}

unsafe impl Send for HipRuntime {}

impl HipRuntime {
    pub fn new(device: i32) -> Result<Self, HipError> {
        let mut ctx = std::ptr::null_mut();
        let rc = unsafe { ffi::atlas_hip_init(device as c_int, &mut ctx) };
        match rc {
            ffi::ATLAS_OK => Ok(HipRuntime { ctx }),
            ffi::ATLAS_ERR_NO_DEVICE => Err(HipError::NoDevice),
            ffi::ATLAS_ERR_OUT_OF_MEMORY => Err(HipError::OutOfMemory("context workspace".into())),
            _ => Err(HipError::CommandFailed("context creation failed".into())),
        }
    }

    /// The raw context, for calls through [`ffi`].
    pub fn as_ptr(&self) -> *mut ffi::AtlasHipCtx {
        self.ctx
    }

    fn check(&self, rc: c_int) -> Result<(), HipError> {
        if rc == ffi::ATLAS_OK {
            return Ok(());
        }
        let msg = unsafe {
            let p = ffi::atlas_hip_last_error(self.ctx);
            if p.is_null() { String::new() } else { CStr::from_ptr(p).to_string_lossy().into_owned() }
        };
        Err(match rc {
            ffi::ATLAS_ERR_NO_DEVICE => HipError::NoDevice,
            ffi::ATLAS_ERR_INVALID_INPUT => HipError::InvalidInput(msg),
            ffi::ATLAS_ERR_OUT_OF_MEMORY => HipError::OutOfMemory(msg),
            _ => HipError::CommandFailed(msg),
        })
    }

    pub fn set_reduction(&self, reduction: Reduction) -> Result<(), HipError> {
        let r = match reduction {
            Reduction::Sequential => ffi::ATLAS_REDUCTION_SEQUENTIAL,
            Reduction::Wide => ffi::ATLAS_REDUCTION_WIDE,
            Reduction::Auto => ffi::ATLAS_REDUCTION_AUTO,
        };
        self.check(unsafe { ffi::atlas_hip_set_reduction(self.ctx, r) })
    }

    /// Enqueue on an external `hipStream_t` (null: the context's own stream).
    ///
    /// # Safety
    /// `stream` must be a valid HIP stream of this context's device, alive
    /// for every call enqueued on it.
    pub unsafe fn set_stream(&self, stream: *mut c_void) -> Result<(), HipError> {
        self.check(ffi::atlas_hip_set_stream(self.ctx, stream))
    }

    /// `ResidentCommand::finish` (crates/atlas-metal/src/lib.rs:743-755): wait
    /// for every enqueued op; device-side failures surface here.
    pub fn finish(&self) -> Result<(), HipError> {
        self.check(unsafe { ffi::atlas_hip_sync(self.ctx) })
    }

    pub fn telemetry(&self) -> Result<ffi::AtlasHipTelemetry, HipError> {
        let mut t = ffi::AtlasHipTelemetry::default();
        self.check(unsafe { ffi::atlas_hip_get_telemetry(self.ctx, &mut t) })?;
        Ok(t)
    }

    /// A device buffer of `len` elements (uninitialised).
    pub fn buffer<T: DevicePod>(&self, len: usize) -> Result<DeviceBuffer<'_, T>, HipError> {
        let mut ptr = std::ptr::null_mut();
        let bytes = len.max(1) * std::mem::size_of::<T>();
        self.check(unsafe { ffi::atlas_hip_malloc(self.ctx, bytes, &mut ptr) })?;
        Ok(DeviceBuffer { rt: self, ptr, len, _t: PhantomData })
    }

    /// `buffer_from_slice` (crates/atlas-metal/src/lib.rs:1975-2054).
    pub fn upload<T: DevicePod>(&self, data: &[T]) -> Result<DeviceBuffer<'_, T>, HipError> {
        let b = self.buffer::<T>(data.len())?;
        let bytes = std::mem::size_of_val(data);
        self.check(unsafe { ffi::atlas_hip_upload(self.ctx, b.ptr, data.as_ptr() as *const c_void, bytes) })?;
        Ok(b)
    }

    // -- resident fused ops: one per reference dispatch -----------------------
    // Each checks its buffers' lengths against the elements the kernel
    // touches (InvalidInput otherwise) before the call; the library checks
    // the shapes themselves.

    /// `rms_norm_f32` / `rms_norm_decode_batch_f32` (kernels.metal:106-133).
    pub fn rms_norm(&self, x: &DeviceBuffer<f32>, w: &DeviceBuffer<f32>, y: &DeviceBuffer<f32>, rows: u32,
                    hidden: u32, eps: f32) -> Result<(), HipError> {
        let n = extent(&[rows as u64, hidden as u64])?;
        holds(x, n, "x")?;
        holds(y, n, "y")?;
        holds(w, hidden as usize, "weight")?;
        self.check(unsafe { ffi::atlas_hip_rms_norm_f32(self.ctx, x.ptr(), w.ptr(), y.ptr_mut(), rows, hidden, eps) })
    }

    /// `gemma4_rms_residual_f32` (kernels.metal:183-214): n = norm(x) * w,
    /// [normalized = n], out = residual + n.  `out` may be `residual` and
    /// `normalized` may be `x`, as at gemma4_executor.rs:4492-4506.
    #[allow(clippy::too_many_arguments)]
    pub fn rms_norm_residual(&self, x: &DeviceBuffer<f32>, w: &DeviceBuffer<f32>, residual: &DeviceBuffer<f32>,
                             normalized: Option<&DeviceBuffer<f32>>, out: &DeviceBuffer<f32>, rows: u32,
                             hidden: u32, eps: f32) -> Result<(), HipError> {
        let count = extent(&[rows as u64, hidden as u64])?;
        holds(x, count, "x")?;
        holds(residual, count, "residual")?;
        holds(out, count, "out")?;
        holds(w, hidden as usize, "weight")?;
        if let Some(b) = normalized {
            holds(b, count, "normalized")?;
        }
        let n = normalized.map_or(std::ptr::null_mut(), |b| b.ptr_mut());
        self.check(unsafe {
            ffi::atlas_hip_rms_norm_residual_f32(self.ctx, x.ptr(), w.ptr(), residual.ptr(), n, out.ptr_mut(), rows,
                                                 hidden, eps)
        })
    }

    /// Llama `vector_add_f32` + RMSNorm (executor.rs:1258-1286).
    #[allow(clippy::too_many_arguments)]
    pub fn add_rms_norm(&self, x: &DeviceBuffer<f32>, residual: &DeviceBuffer<f32>, w: &DeviceBuffer<f32>,
                        residual_out: &DeviceBuffer<f32>, y: &DeviceBuffer<f32>, rows: u32, hidden: u32,
                        eps: f32) -> Result<(), HipError> {
        let n = extent(&[rows as u64, hidden as u64])?;
        holds(x, n, "x")?;
        holds(residual, n, "residual")?;
        holds(residual_out, n, "residual_out")?;
        holds(y, n, "y")?;
        holds(w, hidden as usize, "weight")?;
        self.check(unsafe {
            ffi::atlas_hip_add_rms_norm_f32(self.ctx, x.ptr(), residual.ptr(), w.ptr(), residual_out.ptr_mut(),
                                            y.ptr_mut(), rows, hidden, eps)
        })
    }

    /// `gemma4_ple_rms_add_scale_f32` (kernels.metal:228-258): state =
    /// (state + norm(x) * w) * scale[0].
    pub fn rms_norm_add_scale(&self, x: &DeviceBuffer<f32>, w: &DeviceBuffer<f32>, state: &DeviceBuffer<f32>,
                              scale: &DeviceBuffer<f32>, rows: u32, hidden: u32, eps: f32) -> Result<(), HipError> {
        let n = extent(&[rows as u64, hidden as u64])?;
        holds(x, n, "x")?;
        holds(state, n, "state")?;
        holds(w, hidden as usize, "weight")?;
        holds(scale, 1, "scale")?;
        self.check(unsafe {
            ffi::atlas_hip_rms_norm_add_scale_f32(self.ctx, x.ptr(), w.ptr(), state.ptr_mut(), scale.ptr(), rows,
                                                  hidden, eps)
        })
    }

    /// `gemma4_qk_norm_rope_fused_batch_f32` (kernels.metal:1098-1195).
    #[allow(clippy::too_many_arguments)]
    pub fn qk_norm_rope(&self, q: &DeviceBuffer<f32>, k: &DeviceBuffer<f32>, q_weight: &DeviceBuffer<f32>,
                        k_weight: &DeviceBuffer<f32>, cos: &DeviceBuffer<f32>, sin: &DeviceBuffer<f32>,
                        q_out: &DeviceBuffer<f32>, k_out: &DeviceBuffer<f32>, tokens: u32, q_heads: u32,
                        has_key: bool, head_dim: u32, rope_stride: u32, eps: f32) -> Result<(), HipError> {
        let qn = extent(&[tokens as u64, q_heads as u64, head_dim as u64])?;
        holds(q, qn, "q")?;
        holds(q_out, qn, "q_out")?;
        holds(q_weight, head_dim as usize, "q_weight")?;
        if has_key {
            let kn = extent(&[tokens as u64, head_dim as u64])?;
            holds(k, kn, "k")?;
            holds(k_out, kn, "k_out")?;
            holds(k_weight, head_dim as usize, "k_weight")?;
        }
        if tokens > 0 {
            // row t of the tables is read at t * rope_stride, head_dim / 2 pairs
            let rows = extent(&[tokens as u64 - 1, rope_stride as u64])?;
            let tn = rows.checked_add(head_dim as usize / 2).ok_or_else(|| invalid("buffer extent overflows".into()))?;
            holds(cos, tn, "cos")?;
            holds(sin, tn, "sin")?;
        }
        self.check(unsafe {
            ffi::atlas_hip_qk_norm_rope_f32(self.ctx, q.ptr(), k.ptr(), q_weight.ptr(), k_weight.ptr(), cos.ptr(),
                                            sin.ptr(), q_out.ptr_mut(), k_out.ptr_mut(), tokens, q_heads,
                                            has_key as u32, head_dim, rope_stride, eps)
        })
    }

    /// `silu_f32` + `vector_multiply_f32` (kernels.metal:27-36, 64-69).
    pub fn swiglu(&self, gate: &DeviceBuffer<f32>, up: &DeviceBuffer<f32>, out: &DeviceBuffer<f32>, n: u64)
                  -> Result<(), HipError> {
        let count = extent(&[n])?;
        holds(gate, count, "gate")?;
        holds(up, count, "up")?;
        holds(out, count, "out")?;
        self.check(unsafe { ffi::atlas_hip_swiglu_f32(self.ctx, gate.ptr(), up.ptr(), out.ptr_mut(), n) })
    }

    /// `gelu_multiply_f32` (kernels.metal:773-784).
    pub fn geglu(&self, gate: &DeviceBuffer<f32>, up: &DeviceBuffer<f32>, out: &DeviceBuffer<f32>, n: u64)
                 -> Result<(), HipError> {
        let count = extent(&[n])?;
        holds(gate, count, "gate")?;
        holds(up, count, "up")?;
        holds(out, count, "out")?;
        self.check(unsafe { ffi::atlas_hip_geglu_f32(self.ctx, gate.ptr(), up.ptr(), out.ptr_mut(), n) })
    }

    /// `embedding_lookup_f32` (kernels.metal:94-104) [+ scale].
    #[allow(clippy::too_many_arguments)]
    pub fn embed_f32(&self, table: &DeviceBuffer<f32>, ids: &DeviceBuffer<u32>, out: &DeviceBuffer<f32>, vocab: u32,
                     hidden: u32, tokens: u32, scale: f32) -> Result<(), HipError> {
        holds(table, extent(&[vocab as u64, hidden as u64])?, "table")?;
        holds(ids, tokens as usize, "ids")?;
        holds(out, extent(&[tokens as u64, hidden as u64])?, "out")?;
        self.check(unsafe {
            ffi::atlas_hip_embed_f32(self.ctx, table.ptr(), ids.ptr(), out.ptr_mut(), vocab, hidden, tokens, scale)
        })
    }

    /// `embedding_lookup_{q4_0,q8_0,q6_k}` (kernels.metal:653-692) times
    /// `scale` (Gemma: sqrt(hidden), gemma4_executor.rs:4145-4161).
    #[allow(clippy::too_many_arguments)]
    pub fn embed_quant(&self, format: u32, table: &DeviceBuffer<u8>, ids: &DeviceBuffer<u32>,
                       out: &DeviceBuffer<f32>, vocab: u32, hidden: u32, tokens: u32, scale: f32)
                       -> Result<(), HipError> {
        let f = match format {
            ffi::ATLAS_GGUF_Q4_0 => ffi::atlas_hip_embed_q4_0,
            ffi::ATLAS_GGUF_Q8_0 => ffi::atlas_hip_embed_q8_0,
            ffi::ATLAS_GGUF_Q6_K => ffi::atlas_hip_embed_q6_k,
            other => return Err(HipError::InvalidInput(format!("unsupported packed embedding format {other}"))),
        };
        let row = packed_row_bytes(format, hidden).unwrap_or(0);
        holds(table, extent(&[vocab as u64, row])?, "table")?;
        holds(ids, tokens as usize, "ids")?;
        holds(out, extent(&[tokens as u64, hidden as u64])?, "out")?;
        self.check(unsafe { f(self.ctx, table.ptr(), ids.ptr(), out.ptr_mut(), vocab, hidden, tokens, scale) })
    }

    /// The Gemma PLE chain (gemma4_executor.rs:4162-4237).
    #[allow(clippy::too_many_arguments)]
    pub fn ple(&self, q6_k: bool, table: &DeviceBuffer<u8>, ids: &DeviceBuffer<u32>, projection: &DeviceBuffer<f32>,
               out: &DeviceBuffer<f32>, vocab: u32, layers: u32, width: u32, tokens: u32, embedding_scale: f32,
               output_scale: f32) -> Result<(), HipError> {
        let f = if q6_k { ffi::atlas_hip_ple_q6_k } else { ffi::atlas_hip_ple_q4_0 };
        let values = extent(&[layers as u64, width as u64])?;
        let fmt = if q6_k { ffi::ATLAS_GGUF_Q6_K } else { ffi::ATLAS_GGUF_Q4_0 };
        let row = u32::try_from(values).ok().and_then(|v| packed_row_bytes(fmt, v)).unwrap_or(0);
        holds(table, extent(&[vocab as u64, row])?, "table")?;
        holds(ids, tokens as usize, "ids")?;
        let n = extent(&[tokens as u64, values as u64])?;
        holds(projection, n, "projection")?;
        holds(out, n, "out")?;
        self.check(unsafe {
            f(self.ctx, table.ptr(), ids.ptr(), projection.ptr(), out.ptr_mut(), vocab, layers, width, tokens,
              embedding_scale, output_scale)
        })
    }
}

impl Drop for HipRuntime {
    fn drop(&mut self) {
        unsafe { ffi::atlas_hip_destroy(self.ctx) }
    }
}

/// A device allocation of `len` elements of `T`, freed on drop: `GpuBuffer`.
pub struct DeviceBuffer<'rt, T: DevicePod> {
    rt: &'rt HipRuntime,
    ptr: *mut c_void,
    len: usize,
    _t: PhantomData<T>,
}

impl<T: DevicePod> DeviceBuffer<'_, T> {
    pub fn len(&self) -> usize {
        self.len
    }
    pub fn is_empty(&self) -> bool {
        self.len == 0
    }
    pub fn ptr(&self) -> *const T {
        self.ptr as *const T
    }
    pub fn ptr_mut(&self) -> *mut T {
        self.ptr as *mut T
    }

    /// Synchronous read-back (`GpuBuffer` contents after `finish`).
    pub fn download(&self) -> Result<Vec<T>, HipError> {
        let mut out = Vec::with_capacity(self.len);
        let bytes = self.len * std::mem::size_of::<T>();
        self.rt.check(unsafe { ffi::atlas_hip_download(self.rt.ctx, out.as_mut_ptr() as *mut c_void, self.ptr, bytes) })?;
        unsafe { out.set_len(self.len) };
        Ok(out)
    }
}

impl<T: DevicePod> Drop for DeviceBuffer<'_, T> {
    fn drop(&mut self) {
        unsafe {
            ffi::atlas_hip_free(self.rt.ctx, self.ptr);
        }
    }
}

/// `atlas_ops::NeuralOps` (crates/atlas-ops/src/lib.rs:20-147) over the HIP
/// library: each call validates, copies in, runs, waits and copies out.
pub struct NeuralOps {
    runtime: HipRuntime,
}

macro_rules! host_call {
    ($self:ident, $len:expr, |$out:ident, $t:ident| $call:expr) => {{
        let mut $out = vec![0.0f32; $len];
        let mut $t = ffi::AtlasDispatchTiming::default();
        $self.runtime.check(unsafe { $call })?;
        Ok(($out, DispatchTiming::from($t)))
    }};
}

impl NeuralOps {
    pub fn new() -> Result<Self, OperatorError> {
        Ok(Self { runtime: HipRuntime::new(0)? })
    }
    pub fn runtime(&self) -> &HipRuntime {
        &self.runtime
    }
    fn ctx(&self) -> *mut ffi::AtlasHipCtx {
        self.runtime.ctx
    }

    pub fn embedding(&self, table: &[f32], vocabulary: usize, hidden: usize, token_ids: &[u32])
                     -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, token_ids.len() * hidden, |out, t| ffi::atlas_ops_embedding(
            self.ctx(), table.as_ptr(), table.len(), vocabulary, hidden, token_ids.as_ptr(), token_ids.len(),
            out.as_mut_ptr(), out.len(), &mut t))
    }
    pub fn add(&self, lhs: &[f32], rhs: &[f32]) -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, lhs.len(), |out, t| ffi::atlas_ops_add(
            self.ctx(), lhs.as_ptr(), lhs.len(), rhs.as_ptr(), rhs.len(), out.as_mut_ptr(), out.len(), &mut t))
    }
    pub fn multiply(&self, lhs: &[f32], rhs: &[f32]) -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, lhs.len(), |out, t| ffi::atlas_ops_multiply(
            self.ctx(), lhs.as_ptr(), lhs.len(), rhs.as_ptr(), rhs.len(), out.as_mut_ptr(), out.len(), &mut t))
    }
    pub fn silu(&self, input: &[f32]) -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, input.len(), |out, t| ffi::atlas_ops_silu(
            self.ctx(), input.as_ptr(), input.len(), out.as_mut_ptr(), out.len(), &mut t))
    }
    pub fn rms_norm(&self, input: &[f32], rows: usize, hidden: usize, weight: &[f32], epsilon: f32)
                    -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, input.len(), |out, t| ffi::atlas_ops_rms_norm(
            self.ctx(), input.as_ptr(), input.len(), rows, hidden, weight.as_ptr(), weight.len(), epsilon,
            out.as_mut_ptr(), out.len(), &mut t))
    }
    pub fn rope(&self, input: &[f32], rows: usize, hidden: usize, cos: &[f32], sin: &[f32])
                -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, input.len(), |out, t| ffi::atlas_ops_rope(
            self.ctx(), input.as_ptr(), input.len(), rows, hidden, cos.as_ptr(), cos.len(), sin.as_ptr(), sin.len(),
            out.as_mut_ptr(), out.len(), &mut t))
    }
    /// `MetalRuntime::gelu` (crates/atlas-metal/src/lib.rs:1913-1926).
    pub fn gelu(&self, input: &[f32]) -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, input.len(), |out, t| ffi::atlas_ops_gelu(
            self.ctx(), input.as_ptr(), input.len(), out.as_mut_ptr(), out.len(), &mut t))
    }
    /// `MetalRuntime::embedding_lookup_q6_k` (crates/atlas-metal/src/lib.rs:1437-1483).
    pub fn embedding_q6_k(&self, weights: &[u8], vocabulary: usize, hidden: usize, token_ids: &[u32])
                          -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, token_ids.len() * hidden, |out, t| ffi::atlas_ops_embedding_q6_k(
            self.ctx(), weights.as_ptr(), weights.len(), vocabulary, hidden, token_ids.as_ptr(), token_ids.len(),
            out.as_mut_ptr(), out.len(), &mut t))
    }
    /// `MetalRuntime::scalar_multiply` (crates/atlas-metal/src/lib.rs:1348-1366).
    pub fn scalar_multiply(&self, input: &[f32], scalar: f32) -> Result<(Vec<f32>, DispatchTiming), OperatorError> {
        host_call!(self, input.len(), |out, t| ffi::atlas_ops_scalar_multiply(
            self.ctx(), input.as_ptr(), input.len(), scalar, out.as_mut_ptr(), out.len(), &mut t))
    }
}

/// Host RoPE tables: `gemma4_rope_angle` (gemma4_executor.rs:622-633) per
/// token position and pair, `[tokens][rope_pairs]` cos and sin.
pub fn rope_tables_gemma4(positions: &[u32], rope_pairs: usize, rotary: usize, theta: f32,
                          frequency_factors: Option<&[f32]>) -> Result<(Vec<f32>, Vec<f32>), HipError> {
    let n = positions.len() * rope_pairs;
    let (mut c, mut s) = (vec![0.0f32; n], vec![0.0f32; n]);
    let ff = frequency_factors.map_or(std::ptr::null(), |f| f.as_ptr());
    let rc = unsafe {
        ffi::atlas_rope_tables_gemma4(positions.as_ptr(), positions.len(), rope_pairs, rotary, theta, ff,
                                      c.as_mut_ptr(), s.as_mut_ptr())
    };
    if rc != ffi::ATLAS_OK {
        return Err(HipError::InvalidInput("RoPE table dimensions are invalid".into()));
    }
    Ok((c, s))
}

/// A GGUF model memory-mapped by the library (`GgufModel::open`,
/// crates/atlas-core/src/gguf.rs:112-225).
pub struct GgufModel {
    raw: *mut ffi::AtlasGguf,
}

impl GgufModel {
    pub fn open(path: &str) -> Result<Self, HipError> {
        let c = CString::new(path).map_err(|_| HipError::InvalidInput("path holds a NUL byte".into()))?;
        let mut raw = std::ptr::null_mut();
        let mut err = vec![0 as std::os::raw::c_char; 512];
        let rc = unsafe { ffi::atlas_gguf_open(c.as_ptr(), &mut raw, err.as_mut_ptr(), err.len()) };
        if rc != ffi::ATLAS_OK {
            let msg = unsafe { CStr::from_ptr(err.as_ptr()) }.to_string_lossy().into_owned();
            return Err(HipError::InvalidInput(msg));
        }
        Ok(GgufModel { raw })
    }
    pub fn as_ptr(&self) -> *const ffi::AtlasGguf {
        self.raw
    }
    pub fn tensor_count(&self) -> u64 {
        unsafe { ffi::atlas_gguf_tensor_count(self.raw) }
    }
    pub fn find_tensor(&self, name: &str) -> Option<u64> {
        let c = CString::new(name).ok()?;
        let i = unsafe { ffi::atlas_gguf_find_tensor(self.raw, c.as_ptr()) };
        if i < 0 { None } else { Some(i as u64) }
    }
    /// Copy tensor `index`'s encoded bytes into a fresh device buffer (the
    /// upload of `ensure_resident_weights`, crates/atlas-model/src/lib.rs:720-753).
    pub fn upload<'rt>(&self, rt: &'rt HipRuntime, index: u64) -> Result<DeviceBuffer<'rt, u8>, HipError> {
        let mut info = std::mem::MaybeUninit::<ffi::AtlasGgufTensor>::uninit();
        rt.check(unsafe { ffi::atlas_gguf_tensor_info(self.raw, index, info.as_mut_ptr()) })?;
        let info = unsafe { info.assume_init() };
        let buf = rt.buffer::<u8>(info.bytes as usize)?;
        rt.check(unsafe { ffi::atlas_gguf_upload_tensor(rt.ctx, self.raw, index, buf.ptr) })?;
        Ok(buf)
    }
}

impl Drop for GgufModel {
    fn drop(&mut self) {
        unsafe { ffi::atlas_gguf_close(self.raw) }
    }
}
