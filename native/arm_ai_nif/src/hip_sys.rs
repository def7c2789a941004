//! The few HIP runtime calls the NIF makes itself (libamdhip64): device
//! buffers for the model's f32 tensors and decode-step state, copies on the
//! library context's stream, and the HIP graph of the decode step.
#![allow(non_camel_case_types, non_upper_case_globals, dead_code)]
use std::os::raw::{c_char, c_int, c_uint, c_void};

pub type hipError_t = c_int;
pub type hipStream_t = *mut c_void;
pub type hipGraph_t = *mut c_void;
pub type hipGraphExec_t = *mut c_void;

pub const hipSuccess: hipError_t = 0;
pub const hipMemcpyHostToDevice: c_int = 1;
pub const hipMemcpyDeviceToHost: c_int = 2;
pub const hipStreamCaptureModeThreadLocal: c_int = 1;
pub const hipHostMallocDefault: c_uint = 0;

extern "C" {
    pub fn hipSetDevice(device: c_int) -> hipError_t;
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> hipError_t;
    pub fn hipFree(ptr: *mut c_void) -> hipError_t;
    pub fn hipHostMalloc(ptr: *mut *mut c_void, size: usize, flags: c_uint) -> hipError_t;
    pub fn hipHostFree(ptr: *mut c_void) -> hipError_t;
    pub fn hipMemcpyAsync(dst: *mut c_void, src: *const c_void, bytes: usize, kind: c_int,
                          stream: hipStream_t) -> hipError_t;
    pub fn hipStreamSynchronize(stream: hipStream_t) -> hipError_t;
    pub fn hipStreamBeginCapture(stream: hipStream_t, mode: c_int) -> hipError_t;
    pub fn hipStreamEndCapture(stream: hipStream_t, graph: *mut hipGraph_t) -> hipError_t;
    pub fn hipGraphInstantiate(exec: *mut hipGraphExec_t, graph: hipGraph_t, error_node: *mut *mut c_void,
                               log: *mut c_char, log_size: usize) -> hipError_t;
    pub fn hipGraphLaunch(exec: hipGraphExec_t, stream: hipStream_t) -> hipError_t;
    pub fn hipGraphExecDestroy(exec: hipGraphExec_t) -> hipError_t;
    pub fn hipGraphDestroy(graph: hipGraph_t) -> hipError_t;
    pub fn hipGetErrorString(e: hipError_t) -> *const c_char;
}

pub fn hip_check(e: hipError_t, what: &str) -> Result<(), String> {
    if e == hipSuccess {
        Ok(())
    } else {
        let msg = unsafe { std::ffi::CStr::from_ptr(hipGetErrorString(e)) }.to_string_lossy().into_owned();
        Err(format!("{what}: {msg}"))
    }
}

/// Device memory of `bytes` bytes, freed on drop.
pub struct DeviceBuf {
    pub ptr: *mut c_void,
    pub bytes: usize,
}

unsafe impl Send for DeviceBuf {}

impl DeviceBuf {
    pub fn new(bytes: usize) -> Result<Self, String> {
        let mut ptr = std::ptr::null_mut();
        hip_check(unsafe { hipMalloc(&mut ptr, bytes.max(256)) }, "hipMalloc")?;
        Ok(Self { ptr, bytes })
    }
    /// A device copy of `data`, complete when the stream reaches this point.
    pub fn from_slice<T: Copy>(data: &[T], stream: hipStream_t) -> Result<Self, String> {
        let bytes = std::mem::size_of_val(data);
        let b = Self::new(bytes)?;
        hip_check(unsafe { hipMemcpyAsync(b.ptr, data.as_ptr() as *const c_void, bytes, hipMemcpyHostToDevice,
                                          stream) }, "hipMemcpyAsync H2D")?;
        // the source is a borrowed host slice: finish the copy before returning
        hip_check(unsafe { hipStreamSynchronize(stream) }, "hipStreamSynchronize")?;
        Ok(b)
    }
    pub fn f32(&self) -> *mut f32 {
        self.ptr as *mut f32
    }
    pub fn i64(&self) -> *mut i64 {
        self.ptr as *mut i64
    }
    /// Byte offset into the buffer, as f32 pointer.
    pub fn f32_at(&self, elems: usize) -> *mut f32 {
        debug_assert!(elems * 4 <= self.bytes);
        unsafe { (self.ptr as *mut f32).add(elems) }
    }
}

impl Drop for DeviceBuf {
    fn drop(&mut self) {
        unsafe {
            hipFree(self.ptr);
        }
    }
}

/// Pinned host memory for the per-token read-back.
pub struct PinnedBuf {
    pub ptr: *mut c_void,
    pub bytes: usize,
}

unsafe impl Send for PinnedBuf {}

impl PinnedBuf {
    pub fn new(bytes: usize) -> Result<Self, String> {
        let mut ptr = std::ptr::null_mut();
        hip_check(unsafe { hipHostMalloc(&mut ptr, bytes.max(64), hipHostMallocDefault) }, "hipHostMalloc")?;
        Ok(Self { ptr, bytes })
    }
    pub fn i64_slice(&self, n: usize) -> &[i64] {
        assert!(n * 8 <= self.bytes);
        unsafe { std::slice::from_raw_parts(self.ptr as *const i64, n) }
    }
}

impl Drop for PinnedBuf {
    fn drop(&mut self) {
        unsafe {
            hipHostFree(self.ptr);
        }
    }
}
