//! Errors of the HIP sampler library: a status code per call and the
//! message of the last failure on the calling thread.
use std::cell::RefCell;
use std::ffi::{CStr, c_char, c_void};
use std::fmt;
use std::sync::Once;

use crate::ffi;

static INSTALL: Once = Once::new();

// The library stores its last error per thread and calls the handler on the
// failing call's own thread, so the Rust slot is per thread too.
thread_local! {
    static LAST_ERROR: RefCell<Option<String>> = const { RefCell::new(None) };
}

/// A failed library call: its `AXS_E_*` status and message.
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct HipSamplerError {
    pub status: i32,
    pub message: String,
}

impl fmt::Display for HipSamplerError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "ax_hip_sampler error {}: {}", self.status, self.message)
    }
}

impl std::error::Error for HipSamplerError {}

unsafe extern "C" fn recording_error_handler(msg: *const c_char, _data: *mut c_void) {
    // Runs inside the library's C++ frames: must not unwind.
    let message = if msg.is_null() {
        String::from("unknown ax_hip_sampler error")
    } else {
        unsafe { CStr::from_ptr(msg) }.to_string_lossy().into_owned()
    };
    let _ = LAST_ERROR.try_with(|slot| *slot.borrow_mut() = Some(message));
}

/// Registers the recording error handler with the library.  Idempotent.
pub fn install_recoverable_error_handler() {
    INSTALL.call_once(|| unsafe {
        ffi::axs_set_error_handler(Some(recording_error_handler), std::ptr::null_mut());
    });
}

/// Takes this thread's recorded error message, if any.
pub fn take_last_error() -> Option<String> {
    LAST_ERROR.try_with(|slot| slot.borrow_mut().take()).ok().flatten()
}

/// `Ok` for `AXS_OK`, else the status with this thread's message.
pub(crate) fn check(status: i32) -> Result<(), HipSamplerError> {
    if status == ffi::AXS_OK as i32 {
        return Ok(());
    }
    let message = take_last_error().unwrap_or_else(|| unsafe {
        let p = ffi::axs_last_error();
        if p.is_null() { String::new() } else { CStr::from_ptr(p).to_string_lossy().into_owned() }
    });
    Err(HipSamplerError { status, message })
}
