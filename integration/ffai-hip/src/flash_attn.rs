//! The device counterparts of `ffai_mercury::asr::flash_attn::{serves, attend, attend_merged}`
//! (crates/ffai-mercury/src/asr/flash_attn.rs:103-129, :131-158, :212-264), with the same
//! names, argument meaning and decline contract: `Ok(None)` where the reference returns
//! `Ok(None)` (the caller then takes its three-op path), `Err` where it bails.
//!
//! The reference's ops allocate their output (`cpu_fwd`, :193, :316, :369); here the caller's
//! HIP backend allocates it and passes a view, together with a workspace from its pool (zeroed
//! once when the pool allocates it) and the stream the call is ordered on.

use std::ffi::CStr;
use std::os::raw::c_void;

use crate::ffi;

/// Element types the kernels take.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum DType {
    F32,
    F16,
    BF16,
}

impl DType {
    const fn code(self) -> i32 {
        match self {
            Self::F32 => ffi::FFAI_F32,
            Self::F16 => ffi::FFAI_F16,
            Self::BF16 => ffi::FFAI_BF16,
        }
    }
}

/// A 4-D view of device memory: element (0,0,0,0) at `ptr`, strides in elements.
#[derive(Clone, Copy, Debug)]
pub struct DeviceView {
    pub ptr: *mut c_void,
    pub dtype: DType,
    pub dims: [i64; 4],
    pub strides: [i64; 4],
}

impl DeviceView {
    /// A contiguous view of `dims`.
    pub fn contiguous(ptr: *mut c_void, dtype: DType, dims: [i64; 4]) -> Self {
        let strides = [dims[1] * dims[2] * dims[3], dims[2] * dims[3], dims[3], 1];
        Self { ptr, dtype, dims, strides }
    }

    fn raw(&self) -> ffi::ffai_tensor {
        ffi::ffai_tensor {
            data: self.ptr,
            dtype: self.dtype.code(),
            on_device: 1,
            dims: self.dims,
            strides: self.strides,
        }
    }
}

/// A device workspace from the caller's pool: `bytes` at `ptr`, zeroed once when allocated
/// (every call leaves its split counters zero again).
#[derive(Clone, Copy, Debug)]
pub struct Workspace {
    pub ptr: *mut c_void,
    pub bytes: usize,
}

impl Workspace {
    pub const fn none() -> Self {
        Self { ptr: std::ptr::null_mut(), bytes: 0 }
    }
}

/// A negative status of the C ABI with `ffai_attn_last_error`'s description: the reference's
/// `candle::Error` from its `bail!`s.
#[derive(Clone, Debug)]
pub struct FfaiError {
    pub code: i32,
    pub message: String,
}

impl std::fmt::Display for FfaiError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "ffai_attn error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for FfaiError {}

fn last_error(code: i32) -> FfaiError {
    // SAFETY: the library returns a NUL-terminated thread-local string that stays valid until
    // the next call on this thread; it is copied at once.
    let message = unsafe { CStr::from_ptr(ffi::ffai_attn_last_error()) }
        .to_string_lossy()
        .into_owned();
    FfaiError { code, message }
}

/// OK -> Some(()), DECLINED -> None, negative -> Err.
fn status(rc: i32) -> Result<Option<()>, FfaiError> {
    match rc {
        ffi::FFAI_OK => Ok(Some(())),
        ffi::FFAI_DECLINED => Ok(None),
        code => Err(last_error(code)),
    }
}

/// `flash_attn::serves` (:103-129): whether `attend` takes these K^T (1,H,64,K) and V (1,H,K,64)
/// at decode, with the same key floor as the kernel (`set_decode_min_keys`).
pub fn serves(kt: &DeviceView, v: &DeviceView) -> bool {
    let (a, b) = (kt.raw(), v.raw());
    // SAFETY: both views are plain values; the function only reads them.
    unsafe { ffi::ffai_serves(&a, &b) == 1 }
}

/// Workspace `attend` needs for these operands; `Ok(None)` where `attend` declines.
pub fn attend_workspace_bytes(q: &DeviceView, kt: &DeviceView, v: &DeviceView)
                              -> Result<Option<usize>, FfaiError> {
    let (a, b, c) = (q.raw(), kt.raw(), v.raw());
    let mut bytes = 0usize;
    // SAFETY: views are read; `bytes` is a valid out-pointer.
    let rc = unsafe { ffi::ffai_attend_workspace_bytes(&a, &b, &c, &mut bytes) };
    Ok(status(rc)?.map(|()| bytes))
}

/// `flash_attn::attend` (:212-264): q (1,H,qlen,64) f32, kt (1,H,64,K) and v (1,H,K,64) f32
/// (or f16 at qlen 1), into `out` (1,H,qlen,64) f32. `Ok(None)`: declined, exactly where the
/// reference declines (masked, shapes, dtype, key floor).
pub fn attend(q: &DeviceView, kt: &DeviceView, v: &DeviceView, masked: bool, out: &DeviceView,
              workspace: Workspace, stream: *mut c_void) -> Result<Option<()>, FfaiError> {
    let (a, b, c) = (q.raw(), kt.raw(), v.raw());
    let mut o = out.raw();
    // SAFETY: every pointer in the views is device memory of the stated extent, owned by the
    // caller for the duration of the stream-ordered call.
    status(unsafe {
        ffi::ffai_attend(&a, &b, &c, i32::from(masked), &mut o, workspace.ptr, workspace.bytes,
                         stream)
    })
}

/// Workspace `attend_merged` needs; `Ok(None)` where it declines.
pub fn attend_merged_workspace_bytes(q: &DeviceView, kt: &DeviceView, v: &DeviceView)
                                     -> Result<Option<usize>, FfaiError> {
    let (a, b, c) = (q.raw(), kt.raw(), v.raw());
    let mut bytes = 0usize;
    // SAFETY: views are read; `bytes` is a valid out-pointer.
    let rc = unsafe { ffi::ffai_attend_merged_workspace_bytes(&a, &b, &c, &mut bytes) };
    Ok(status(rc)?.map(|()| bytes))
}

/// `flash_attn::attend_merged` (:131-158): encoder attention into the merged (1,T,H*64) f32
/// layout.
pub fn attend_merged(q: &DeviceView, kt: &DeviceView, v: &DeviceView, out: &DeviceView,
                     workspace: Workspace, stream: *mut c_void)
                     -> Result<Option<()>, FfaiError> {
    let (a, b, c) = (q.raw(), kt.raw(), v.raw());
    let mut o = out.raw();
    // SAFETY: as for `attend`.
    status(unsafe {
        ffi::ffai_attend_merged(&a, &b, &c, &mut o, workspace.ptr, workspace.bytes, stream)
    })
}

/// One general call (batch, GQA, bf16/f16/f32, head_dim 64/128, causal with offset, ragged
/// keys): the descriptor path the mirrors dispatch through.
pub struct Attention {
    desc: ffi::ffai_attn_desc,
}

impl Attention {
    /// Contiguous operands: q (batch, heads_q, q_len, head_dim); K as `k_layout` says; V
    /// (batch, heads_kv, kv_len, head_dim); out like q.
    #[allow(clippy::too_many_arguments)]
    pub fn new(q_dtype: DType, kv_dtype: DType, out_dtype: DType, batch: i32, heads_q: i32,
               heads_kv: i32, q_len: i32, kv_len: i32, head_dim: i32, k_transposed: bool)
               -> Self {
        let mut desc = std::mem::MaybeUninit::<ffi::ffai_attn_desc>::uninit();
        // SAFETY: ffai_attn_desc_init writes every field of the descriptor.
        let desc = unsafe {
            ffi::ffai_attn_desc_init(desc.as_mut_ptr(), q_dtype.code(), kv_dtype.code(),
                                     out_dtype.code(), batch, heads_q, heads_kv, q_len, kv_len,
                                     head_dim,
                                     if k_transposed { ffi::FFAI_K_TRANSPOSED } else { ffi::FFAI_K_ROWS });
            desc.assume_init()
        };
        Self { desc }
    }

    pub fn scale(mut self, scale: f32) -> Self {
        self.desc.scale = scale;
        self
    }

    /// Key j hidden from query i iff j > q_offset + i.
    pub fn causal(mut self, q_offset: i32) -> Self {
        self.desc.causal = 1;
        self.desc.q_offset = q_offset;
        self
    }

    /// Device int32[batch]: keys valid per batch item.
    pub fn kv_lens(mut self, lens: *const i32) -> Self {
        self.desc.kv_lens = lens;
        self
    }

    /// Element strides of q, k, v, out (batch, head, row, column); a batch stride of 0 on K/V
    /// shares one cache across the batch (beam cross-attention).
    pub fn strides(mut self, q: [i64; 4], k: [i64; 4], v: [i64; 4], o: [i64; 4]) -> Self {
        self.desc.q_strides = q;
        self.desc.k_strides = k;
        self.desc.v_strides = v;
        self.desc.o_strides = o;
        self
    }

    pub fn serves(&self) -> bool {
        // SAFETY: the descriptor is read.
        unsafe { ffi::ffai_attn_serves(&self.desc) == 1 }
    }

    pub fn workspace_bytes(&self) -> Result<Option<usize>, FfaiError> {
        let mut bytes = 0usize;
        // SAFETY: the descriptor is read; `bytes` is a valid out-pointer.
        let rc = unsafe { ffi::ffai_attn_workspace_bytes(&self.desc, &mut bytes) };
        Ok(status(rc)?.map(|()| bytes))
    }

    /// Run on `stream`; `Ok(None)` where the descriptor is not served.
    pub fn run(&self, q: *const c_void, k: *const c_void, v: *const c_void, out: *mut c_void,
               workspace: Workspace, stream: *mut c_void) -> Result<Option<()>, FfaiError> {
        // SAFETY: the pointers are device memory of the extents the descriptor states.
        status(unsafe {
            ffi::ffai_attn_fwd(&self.desc, q, k, v, out, workspace.ptr, workspace.bytes, stream)
        })
    }
}

/// Mirror of `knobs::DECODE_MIN_KEYS` (knobs.rs:163-168).
pub fn decode_min_keys() -> i32 {
    // SAFETY: reads an atomic in the library.
    unsafe { ffi::ffai_get_decode_min_keys() }
}

pub fn set_decode_min_keys(n: i32) {
    // SAFETY: writes an atomic in the library.
    unsafe { ffi::ffai_set_decode_min_keys(n) }
}
