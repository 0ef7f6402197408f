//! Safe layer over `swiftllm-hip-sys`: the same `CudaError`, `Result` and
//! `bindings::*` items that `crates/swiftllm-cuda` exports for the decode
//! path (lib.rs:16-42, bindings.rs:8-242), so a crate that depends on
//! `swiftllm-cuda` for these items can depend on this one instead.
//!
//! Only the paged-attention path is here: prefill, decode, the cache write,
//! block copies and swaps, MoE routing / dispatch / expert computation. The
//! other stubs of bindings.rs (norms, rotary, activations, quantized GEMMs,
//! sampling) are outside it.

pub mod bindings;

use thiserror::Error;

/// The error type of crates/swiftllm-cuda/src/lib.rs:16-42, variant for
/// variant. The library's status code selects the variant (the negated
/// declaration index) and its message fills the String payload.
#[derive(Error, Debug)]
pub enum CudaError {
    #[error("CUDA initialization failed: {0}")]
    InitError(String),
    #[error("Kernel launch failed: {0}")]
    KernelError(String),
    #[error("Memory allocation failed: {0}")]
    MemoryError(String),
    #[error("Invalid parameter: {0}")]
    InvalidParameter(String),
    #[error("CUDA device not found")]
    DeviceNotFound,
    #[error("Operation not supported: {0}")]
    NotSupported(String),
}

pub type Result<T> = std::result::Result<T, CudaError>;

/// Maps a status of the C ABI onto `Result`.
pub(crate) fn check(status: i32) -> Result<()> {
    use swiftllm_hip_sys as sys;
    if status == sys::SWIFTLLM_OK {
        return Ok(());
    }
    let msg = unsafe { std::ffi::CStr::from_ptr(sys::swiftllm_hip_last_error_message()) }
        .to_string_lossy()
        .into_owned();
    Err(match status {
        sys::SWIFTLLM_ERR_INIT => CudaError::InitError(msg),
        sys::SWIFTLLM_ERR_MEMORY => CudaError::MemoryError(msg),
        sys::SWIFTLLM_ERR_INVALID_PARAMETER => CudaError::InvalidParameter(msg),
        sys::SWIFTLLM_ERR_DEVICE_NOT_FOUND => CudaError::DeviceNotFound,
        sys::SWIFTLLM_ERR_NOT_SUPPORTED => CudaError::NotSupported(msg),
        _ => CudaError::KernelError(msg),
    })
}

