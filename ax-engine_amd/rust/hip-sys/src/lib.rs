//! FFI boundary of the MI355X (gfx950) token sampler, a sibling of
//! `crates/mlx-sys` in the AX Engine workspace.
//!
//! The raw bindings ([`ffi`], bindgen over `include/ax_hip_sampler.h`) and the
//! safe wrapper ([`HipSamplerContext`]) live here, as `mlx-sys` keeps its raw
//! bindings and safe layer together.  Every call returns a status; a failed
//! call's message is kept per thread ([`take_last_error`]) and, once
//! [`install_recoverable_error_handler`] has run, also recorded by the
//! library's error-handler hook on the calling thread (the convention of
//! `mlx_set_error_handler` in crates/mlx-sys/native/ax_shim.h:106-110).
#![allow(unsafe_code)]

pub mod context;
pub mod error;
pub mod philox;

/// Raw bindgen output for `ax_hip_sampler.h`.  Prefer [`HipSamplerContext`].
#[doc(hidden)]
#[allow(non_camel_case_types, non_snake_case, non_upper_case_globals, dead_code, clippy::all)]
pub mod ffi {
    include!(concat!(env!("OUT_DIR"), "/bindings.rs"));
}

pub use context::{HipSamplerContext, HostBatch, HostRowOutputs, RowParams};
pub use error::{HipSamplerError, install_recoverable_error_handler, take_last_error};
