//! darkforest-hip: the C-ABI FFI crate of libdfattn, the MI355X (gfx950) attention library that
//! replaces the attention object of `darkforest-cuda` (darkforest-cuda/build.rs:143-217,
//! src/kernels.rs:689-885).
//!
//! * [`ffi`] declares every entry point of `include/dfattn.h`, [`gpt2`] every one of
//!   `include/dfgpt2.h`; `build.rs` builds the library with hipcc (`make -C
//!   dark-forest_amd/csrc`) and links it and the HIP runtime.
//! * The wrappers below keep the names, argument meaning and error behaviour of the reference's
//!   `kernels.rs` wrappers (`cuda_fused_attention`, `cuda_fused_mha_forward`,
//!   `cuda_attention_backward`, `cuda_fused_mha_backward`, `cuda_sync`): the reference's launchers
//!   run on the null stream and report errors at the next sync, which prints `[darkforest] ...`
//!   and aborts (matmul.cu:21-28).
//! * [`AttentionContext`] owns a `dfattn_context` (lib.rs:1949-2368): its buffers are made at
//!   construction, and the backward reuses the forward's O, lse and fp16 copies when the caller
//!   opts in and passes the same q, k, v.
//!
//! Pointers are device pointers; the caller keeps them valid for the call, as with the reference.

pub mod ffi;
pub mod gpt2;

use std::ffi::CStr;
use std::fmt;
use std::os::raw::{c_int, c_void};

/// A status other than `DFATTN_OK` from a status-returning entry point, with the library's message.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct DfattnError {
    pub status: i32,
    pub message: String,
}

impl fmt::Display for DfattnError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "dfattn error {}: {}", self.status, self.message)
    }
}

impl std::error::Error for DfattnError {}

pub type Result<T> = std::result::Result<T, DfattnError>;

/// `Ok(())` for `DFATTN_OK`, else the status and `dfattn_last_error_message()`.
pub fn check(status: c_int) -> Result<()> {
    if status == ffi::DFATTN_OK {
        return Ok(());
    }
    let message = unsafe {
        let p = ffi::dfattn_last_error_message();
        if p.is_null() { String::new() } else { CStr::from_ptr(p).to_string_lossy().into_owned() }
    };
    Err(DfattnError { status, message })
}

fn dim(x: usize, what: &str) -> Result<u32> {
    u32::try_from(x).map_err(|_| DfattnError { status: ffi::DFATTN_ERR_OVERFLOW, message: format!("{what} = {x} does not fit u32") })
}

/// `cuda_sync` of kernels.rs: waits for the null stream; prints and aborts on a device error or a
/// launcher argument error recorded since the last sync.
pub fn cuda_sync() -> Result<()> {
    unsafe { ffi::darkforest_sync() };
    Ok(())
}

/// `cuda_fused_attention` of kernels.rs:694 (single head, [seq_len, d_head]).
pub fn cuda_fused_attention(q: *const f32, k: *const f32, v: *const f32, out: *mut f32, seq_len: usize,
                            d_head: usize, scale: f32, causal: bool) -> Result<()> {
    unsafe {
        ffi::launch_fused_attention(q, k, v, out, dim(seq_len, "seq_len")?, dim(d_head, "d_head")?, scale,
                                    causal as u32)
    };
    Ok(())
}

/// `cuda_attention_backward` of kernels.rs:735; `probabilities` is the caller's [2, S, S] scratch.
#[allow(clippy::too_many_arguments)]
pub fn cuda_attention_backward(q: *const f32, k: *const f32, v: *const f32, d_out: *const f32, d_q: *mut f32,
                               d_k: *mut f32, d_v: *mut f32, probabilities: *mut f32, seq_len: usize,
                               d_head: usize, scale: f32, causal: bool) -> Result<()> {
    unsafe {
        ffi::launch_attention_backward(q, k, v, d_out, d_q, d_k, d_v, probabilities, dim(seq_len, "seq_len")?,
                                       dim(d_head, "d_head")?, scale, causal as u32)
    };
    Ok(())
}

/// `cuda_fused_mha_forward` of kernels.rs:788 ([seq_len, n_heads * d_head]).
#[allow(clippy::too_many_arguments)]
pub fn cuda_fused_mha_forward(q: *const f32, k: *const f32, v: *const f32, out: *mut f32, n_heads: usize,
                              seq_len: usize, d_head: usize, scale: f32, causal: bool) -> Result<()> {
    unsafe {
        ffi::launch_fused_mha_forward(q, k, v, out, dim(n_heads, "n_heads")?, dim(seq_len, "seq_len")?,
                                      dim(d_head, "d_head")?, scale, causal as u32)
    };
    Ok(())
}

/// `cuda_fused_mha_backward` of kernels.rs:832; `probabilities` is the caller's [H, 2, S, S] scratch,
/// which libdfattn uses as the workspace of its O(H*S*D) backward.
#[allow(clippy::too_many_arguments)]
pub fn cuda_fused_mha_backward(q: *const f32, k: *const f32, v: *const f32, d_out: *const f32, d_q: *mut f32,
                               d_k: *mut f32, d_v: *mut f32, probabilities: *mut f32, n_heads: usize,
                               seq_len: usize, d_head: usize, scale: f32, causal: bool) -> Result<()> {
    unsafe {
        ffi::launch_fused_mha_backward(q, k, v, d_out, d_q, d_k, d_v, probabilities, dim(n_heads, "n_heads")?,
                                       dim(seq_len, "seq_len")?, dim(d_head, "d_head")?, scale, causal as u32)
    };
    Ok(())
}

/// The per-layer attention context (the reference's `AttentionContext`, lib.rs:1949): every buffer
/// is allocated by `new`, the forward writes O and keeps lse, the backward recomputes the forward
/// from the current q, k, v unless `set_reuse_forward(true)` lets it reuse the last forward on the
/// same q, k, v.
pub struct AttentionContext {
    ctx: *mut ffi::DfattnContext,
}

impl AttentionContext {
    /// lib.rs:1981-1989's checks: n_heads, seq_len, d_head >= 1, d_head <= 128.
    pub fn new(n_heads: usize, seq_len: usize, d_head: usize) -> Result<Self> {
        let mut ctx = std::ptr::null_mut();
        check(unsafe {
            ffi::dfattn_context_create(dim(n_heads, "n_heads")?, dim(seq_len, "seq_len")?, dim(d_head, "d_head")?,
                                       &mut ctx)
        })?;
        Ok(Self { ctx })
    }

    pub fn set_reuse_forward(&mut self, enable: bool) -> Result<()> {
        check(unsafe { ffi::dfattn_context_set_reuse_forward(self.ctx, enable as u32) })
    }

    /// The logsumexp [n_heads, seq_len] (device) of the last forward.
    pub fn lse(&self) -> *const f32 {
        unsafe { ffi::dfattn_context_lse(self.ctx) }
    }

    /// `forward_device_into` (lib.rs:2042): O [seq_len, n_heads * d_head] of out_elems floats.
    #[allow(clippy::too_many_arguments)]
    pub fn forward_device_into(&mut self, q: *const f32, k: *const f32, v: *const f32, scale: f32, causal: bool,
                               out: *mut f32, out_elems: usize, stream: *mut c_void) -> Result<()> {
        check(unsafe {
            ffi::dfattn_context_forward_device_into(self.ctx, q, k, v, scale, causal as u32, out, out_elems, stream)
        })
    }

    /// `backward_device_into` (lib.rs:2240): dQ, dK, dV of grad_elems floats each.
    #[allow(clippy::too_many_arguments)]
    pub fn backward_device_into(&mut self, q: *const f32, k: *const f32, v: *const f32, d_out: *const f32,
                                scale: f32, causal: bool, d_q: *mut f32, d_k: *mut f32, d_v: *mut f32,
                                grad_elems: usize, stream: *mut c_void) -> Result<()> {
        check(unsafe {
            ffi::dfattn_context_backward_device_into(self.ctx, q, k, v, d_out, scale, causal as u32, d_q, d_k, d_v,
                                                     grad_elems, stream)
        })
    }
}

impl Drop for AttentionContext {
    fn drop(&mut self) {
        unsafe { ffi::dfattn_context_destroy(self.ctx) };
    }
}

// The context is used from one thread at a time; its device buffers may move between threads.
unsafe impl Send for AttentionContext {}
