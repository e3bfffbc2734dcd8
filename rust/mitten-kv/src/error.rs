//! Status codes of both libraries mapped onto the engine's error type
//! (`inference-backend/src/error.rs:3-13`). The engine aborts the batch on
//! `Err` (`inference-engine/src/engine_loop.rs:47-58`).

use inference_backend::EngineError;
use mitten_kv_sys as sys;
use mitten_kvhost_sys as hsys;
use std::ffi::CStr;

fn message(p: *const std::ffi::c_char) -> String {
    if p.is_null() {
        return String::new();
    }
    // SAFETY: both libraries return a NUL-terminated thread-local string.
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

/// A device-library status: device memory exhaustion is `OutOfKvPages`,
/// everything else `Backend` with the library's message.
pub fn check(status: i32) -> Result<(), EngineError> {
    match status {
        sys::MKV_OK => Ok(()),
        sys::MKV_ERR_OUT_OF_MEMORY => Err(EngineError::OutOfKvPages),
        _ => Err(EngineError::Backend(message(unsafe { sys::mkv_last_error() }))),
    }
}

/// A host-library status: no free block is `OutOfKvPages`.
pub(crate) fn check_host(status: i32) -> Result<(), EngineError> {
    match status {
        hsys::MKVH_OK => Ok(()),
        hsys::MKVH_ERR_EXHAUSTED => Err(EngineError::OutOfKvPages),
        _ => Err(EngineError::Backend(message(unsafe { hsys::mkvh_last_error() }))),
    }
}
