//! The few HIP runtime calls the buffer type needs (libamdhip64).  Streams are passed to the
//! kernels as raw `hipStream_t` handles (`*mut c_void`, null = the null stream).

use std::os::raw::{c_char, c_int, c_void};

pub type HipError = c_int;
pub const HIP_SUCCESS: HipError = 0;

pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

#[link(name = "amdhip64")]
extern "C" {
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> HipError;
    pub fn hipFree(ptr: *mut c_void) -> HipError;
    pub fn hipMemsetAsync(dst: *mut c_void, value: c_int, size: usize, stream: *mut c_void) -> HipError;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> HipError;
    pub fn hipSetDevice(device: c_int) -> HipError;
    pub fn hipStreamSynchronize(stream: *mut c_void) -> HipError;
    pub fn hipGetErrorString(error: HipError) -> *const c_char;
}

/// The runtime's text for a HIP error code.
pub fn error_string(e: HipError) -> String {
    // SAFETY: hipGetErrorString returns a static NUL-terminated string for any code.
    unsafe { std::ffi::CStr::from_ptr(hipGetErrorString(e)) }.to_string_lossy().into_owned()
}
