//! `HipSlice<T>`: a typed device buffer, the HIP stand-in for cudarc's `CudaSlice<T>` and for
//! `vllm_cuda::allocator::DeviceBuffer<T>` (crates/vllm-cuda/src/allocator.rs).

use std::marker::PhantomData;
use std::os::raw::c_void;

use vllm_core::{CoreError, Device, Result as CoreResult};

use crate::hip;

/// Element types the kernels accept, with their `RG_DTYPE_*` code.
pub trait KvElement: Copy + 'static {
    const DTYPE: i32;
}

impl KvElement for f32 {
    const DTYPE: i32 = crate::ffi::RG_DTYPE_F32;
}

/// bfloat16 bits.
#[repr(transparent)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct Bf16(pub u16);

impl KvElement for Bf16 {
    const DTYPE: i32 = crate::ffi::RG_DTYPE_BF16;
}

/// IEEE half bits.
#[repr(transparent)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct F16(pub u16);

impl KvElement for F16 {
    const DTYPE: i32 = crate::ffi::RG_DTYPE_F16;
}

/// `len` elements of `T` in device memory.  Owned buffers (`alloc`, `zeros`) are freed on
/// drop; `from_raw` wraps memory owned elsewhere (a pool view, a framework tensor).
#[derive(Debug)]
pub struct HipSlice<T> {
    ptr: *mut T,
    len: usize,
    owned: bool,
    _t: PhantomData<T>,
}

// SAFETY: a device pointer may be used from any host thread; HIP serialises on the stream.
unsafe impl<T: Send> Send for HipSlice<T> {}
unsafe impl<T: Sync> Sync for HipSlice<T> {}

fn hip_err(what: &str, e: hip::HipError) -> CoreError {
    CoreError::Tensor(format!("{what} failed: {}", hip::error_string(e)))
}

impl<T> HipSlice<T> {
    /// Uninitialised device memory for `len` elements.
    pub fn alloc(len: usize, ordinal: usize) -> CoreResult<Self> {
        let bytes = len * std::mem::size_of::<T>();
        let mut p: *mut c_void = std::ptr::null_mut();
        if bytes > 0 {
            // SAFETY: plain runtime calls with valid out-pointers.
            let e = unsafe { hip::hipSetDevice(ordinal as i32) };
            if e != hip::HIP_SUCCESS {
                return Err(hip_err("hipSetDevice", e));
            }
            let e = unsafe { hip::hipMalloc(&mut p, bytes) };
            if e != hip::HIP_SUCCESS {
                return Err(CoreError::OutOfMemory { device: Device::Cuda(ordinal as u32), requested_bytes: bytes });
            }
        }
        Ok(Self { ptr: p as *mut T, len, owned: true, _t: PhantomData })
    }

    /// Zero-filled device memory (the fill is queued on `stream`).
    pub fn zeros(len: usize, ordinal: usize, stream: *mut c_void) -> CoreResult<Self> {
        let s = Self::alloc(len, ordinal)?;
        if s.byte_len() > 0 {
            // SAFETY: the range was just allocated.
            let e = unsafe { hip::hipMemsetAsync(s.ptr as *mut c_void, 0, s.byte_len(), stream) };
            if e != hip::HIP_SUCCESS {
                return Err(hip_err("hipMemsetAsync", e));
            }
        }
        Ok(s)
    }

    /// Wraps `len` elements at a device address owned elsewhere (not freed on drop).
    ///
    /// # Safety
    /// `ptr` must address at least `len` elements of device memory that outlive the slice.
    pub unsafe fn from_raw(ptr: *mut T, len: usize) -> Self {
        Self { ptr, len, owned: false, _t: PhantomData }
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }

    pub fn byte_len(&self) -> usize {
        self.len * std::mem::size_of::<T>()
    }

    pub fn as_ptr(&self) -> *const c_void {
        self.ptr as *const c_void
    }

    pub fn as_mut_ptr(&mut self) -> *mut c_void {
        self.ptr as *mut c_void
    }

    /// A view of elements `[offset, offset + len)` (e.g. the V half of a fused pool block).
    ///
    /// # Safety
    /// The view must not outlive `self`; writes through it alias `self`.
    pub unsafe fn view(&self, offset: usize, len: usize) -> HipSlice<T> {
        assert!(offset + len <= self.len, "view past the end of the buffer");
        HipSlice::from_raw(self.ptr.add(offset), len)
    }

    /// Synchronous host -> device copy of `src` (`src.len() == self.len()`).
    pub fn copy_from_host(&mut self, src: &[T]) -> CoreResult<()> {
        assert_eq!(src.len(), self.len, "host slice length");
        // SAFETY: both ranges hold byte_len() bytes.
        let e = unsafe {
            hip::hipMemcpy(self.ptr as *mut c_void, src.as_ptr() as *const c_void, self.byte_len(),
                           hip::HIP_MEMCPY_HOST_TO_DEVICE)
        };
        if e != hip::HIP_SUCCESS {
            return Err(hip_err("hipMemcpy", e));
        }
        Ok(())
    }

    /// Synchronous device -> host copy into `dst` (`dst.len() == self.len()`).
    pub fn copy_to_host(&self, dst: &mut [T]) -> CoreResult<()> {
        assert_eq!(dst.len(), self.len, "host slice length");
        // SAFETY: both ranges hold byte_len() bytes.
        let e = unsafe {
            hip::hipMemcpy(dst.as_mut_ptr() as *mut c_void, self.ptr as *const c_void, self.byte_len(),
                           hip::HIP_MEMCPY_DEVICE_TO_HOST)
        };
        if e != hip::HIP_SUCCESS {
            return Err(hip_err("hipMemcpy", e));
        }
        Ok(())
    }
}

impl<T> Drop for HipSlice<T> {
    fn drop(&mut self) {
        if self.owned && !self.ptr.is_null() {
            // SAFETY: owned buffers come from hipMalloc.  A failure here cannot be reported.
            unsafe {
                hip::hipFree(self.ptr as *mut c_void);
            }
        }
    }
}
