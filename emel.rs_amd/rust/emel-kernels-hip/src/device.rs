//! Device plumbing: library status, devices, streams and device buffers.

use core::ffi::{CStr, c_void};
use core::fmt;
use core::marker::PhantomData;
use core::ptr;

use crate::ffi;

/// A status other than `EMEL_OK` from a call whose reference counterpart has
/// no typed error (device management, events the reference does not have).
#[derive(Clone, Copy, Debug, Eq, PartialEq)]
pub struct HipError(pub ffi::Status);

impl HipError {
    /// `Ok(())` for `EMEL_OK`, otherwise the status as an error.
    ///
    /// # Errors
    /// Returns `HipError(status)` for every status other than `EMEL_OK`.
    pub const fn check(status: ffi::Status) -> Result<(), Self> {
        if status == ffi::EMEL_OK { Ok(()) } else { Err(Self(status)) }
    }

    /// The library's fixed text for this status.
    #[must_use]
    pub fn message(self) -> &'static str {
        // SAFETY: emel_status_string returns a static NUL-terminated string
        // for every input.
        let text = unsafe { CStr::from_ptr(ffi::emel_status_string(self.0)) };
        text.to_str().unwrap_or("")
    }
}

impl fmt::Display for HipError {
    fn fmt(&self, formatter: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(formatter, "emel_hip status {}: {}", self.0, self.message())
    }
}

impl std::error::Error for HipError {}

/// The ABI version of the loaded library; [`crate::HipKernel::new`] refuses
/// a library whose version differs from `ffi::EMEL_HIP_ABI_VERSION`.
#[must_use]
pub fn abi_version() -> u32 {
    // SAFETY: no arguments, no preconditions.
    unsafe { ffi::emel_abi_version() }
}

/// Detail of the last failure on the calling thread (empty if none).
#[must_use]
pub fn last_error() -> String {
    // SAFETY: emel_last_error returns a NUL-terminated string owned by the
    // calling thread, valid until its next library call.
    let text = unsafe { CStr::from_ptr(ffi::emel_last_error()) };
    text.to_string_lossy().into_owned()
}

/// Number of visible gfx950 devices.
///
/// # Errors
/// The library status when the HIP runtime cannot be queried.
pub fn device_count() -> Result<i32, HipError> {
    let mut count = 0_i32;
    // SAFETY: `count` is a valid out pointer.
    HipError::check(unsafe { ffi::emel_device_count(&raw mut count) })?;
    Ok(count)
}

/// Makes `device` current for the calling thread.
///
/// # Errors
/// The library status when the device cannot be selected.
pub fn set_device(device: i32) -> Result<(), HipError> {
    // SAFETY: plain value argument.
    HipError::check(unsafe { ffi::emel_set_device(device) })
}

/// Frees the per-stream workspaces the library keeps for reductions and the
/// sampler (they are regrown on demand).
///
/// # Errors
/// The library status when a wait or free fails.
pub fn release_workspaces() -> Result<(), HipError> {
    // SAFETY: no arguments; the library waits for the streams it frees.
    HipError::check(unsafe { ffi::emel_release_workspaces() })
}

/// A HIP stream: either created (and destroyed) by this value or the
/// default stream.
#[derive(Debug)]
pub struct Stream {
    raw: ffi::Stream,
    owned: bool,
}

impl Stream {
    /// Creates a non-blocking stream on the current device.
    ///
    /// # Errors
    /// The library status when the runtime cannot create a stream.
    pub fn new() -> Result<Self, HipError> {
        let mut raw: ffi::Stream = ptr::null_mut();
        // SAFETY: `raw` is a valid out pointer.
        HipError::check(unsafe { ffi::emel_stream_create(&raw mut raw) })?;
        Ok(Self { raw, owned: true })
    }

    /// The device's default (null) stream.
    #[must_use]
    pub const fn default_stream() -> Self {
        Self { raw: ptr::null_mut(), owned: false }
    }

    /// Borrows a `hipStream_t` created elsewhere; it is not destroyed on drop.
    ///
    /// # Safety
    /// `raw` must be a live stream (or null) for as long as the value is used.
    #[must_use]
    pub const unsafe fn from_raw(raw: ffi::Stream) -> Self {
        Self { raw, owned: false }
    }

    /// The `hipStream_t`.
    #[must_use]
    pub const fn as_raw(&self) -> ffi::Stream {
        self.raw
    }

    /// Waits until every launch enqueued on the stream has finished.
    ///
    /// # Errors
    /// The library status when the runtime reports a failure (a failed
    /// kernel included).
    pub fn synchronize(&self) -> Result<(), HipError> {
        // SAFETY: `raw` is live by construction.
        HipError::check(unsafe { ffi::emel_stream_synchronize(self.raw) })
    }

    /// Grows the scratch that calls on this stream share to at least
    /// `work_bytes` of workspace and `counter_bytes` of reduction counters,
    /// so that later calls needing no more allocate nothing (for callers
    /// that capture calls into HIP graphs).
    ///
    /// # Errors
    /// `EMEL_ERR_STREAM_CAPTURE` while the stream is being captured, else
    /// the library status of the allocation.
    pub fn reserve(&self, work_bytes: u64, counter_bytes: u64) -> Result<(), HipError> {
        // SAFETY: `raw` is live by construction.
        HipError::check(unsafe { ffi::emel_stream_reserve(self.raw, work_bytes, counter_bytes) })
    }

    /// The (workspace, counter) bytes this stream's calls share now; after
    /// one eager run of a workload, what to [`Stream::reserve`] for it.
    ///
    /// # Errors
    /// The library status when the current device cannot be read.
    pub fn workspace(&self) -> Result<(u64, u64), HipError> {
        let (mut work, mut counters) = (0u64, 0u64);
        // SAFETY: `raw` is live; both out pointers are valid.
        HipError::check(unsafe { ffi::emel_stream_workspace(self.raw, &raw mut work, &raw mut counters) })?;
        Ok((work, counters))
    }

    /// Builds the current device's lookup tables (GELU's) on this stream and
    /// waits for them, so that no later call waits to build them.
    ///
    /// # Errors
    /// `EMEL_ERR_STREAM_CAPTURE` while the stream is being captured, else
    /// the library status of the build.
    pub fn prepare_device(&self) -> Result<(), HipError> {
        // SAFETY: `raw` is live by construction.
        HipError::check(unsafe { ffi::emel_device_prepare(self.raw) })
    }
}

impl Drop for Stream {
    fn drop(&mut self) {
        if self.owned {
            // SAFETY: created by emel_stream_create and destroyed once.
            let _ = unsafe { ffi::emel_stream_destroy(self.raw) };
        }
    }
}

/// A device allocation of `len` values of `T`, freed on drop.
#[derive(Debug)]
pub struct DeviceBuffer<T: Copy> {
    ptr: *mut T,
    len: usize,
    _owns: PhantomData<T>,
}

impl<T: Copy> DeviceBuffer<T> {
    /// Allocates `len` uninitialised values.
    ///
    /// # Errors
    /// `EMEL_ERR_INVALID_ARGUMENT` when the byte size overflows, else the
    /// library status of the allocation.
    pub fn new(len: usize) -> Result<Self, HipError> {
        let bytes = len.checked_mul(size_of::<T>()).ok_or(HipError(ffi::EMEL_ERR_INVALID_ARGUMENT))?;
        let mut raw: *mut c_void = ptr::null_mut();
        if bytes > 0 {
            // SAFETY: `raw` is a valid out pointer.
            HipError::check(unsafe { ffi::emel_malloc(&raw mut raw, bytes as u64) })?;
        }
        Ok(Self { ptr: raw.cast(), len, _owns: PhantomData })
    }

    /// Allocates a buffer holding a copy of `data`, complete on return.
    ///
    /// # Errors
    /// The library status of the allocation, the copy or the wait.
    pub fn from_host(data: &[T], stream: &Stream) -> Result<Self, HipError> {
        let mut buffer = Self::new(data.len())?;
        buffer.copy_from_host(data, stream)?;
        Ok(buffer)
    }

    /// Copies `data` into the start of the buffer and waits for the copy.
    ///
    /// # Errors
    /// `EMEL_ERR_INVALID_ARGUMENT` when `data` is longer than the buffer,
    /// else the library status of the copy or the wait.
    pub fn copy_from_host(&mut self, data: &[T], stream: &Stream) -> Result<(), HipError> {
        if data.len() > self.len {
            return Err(HipError(ffi::EMEL_ERR_INVALID_ARGUMENT));
        }
        if data.is_empty() {
            return Ok(());
        }
        let bytes = size_of_val(data) as u64;
        // SAFETY: both ranges hold `bytes` bytes; the wait below keeps `data`
        // borrowed until the copy has finished.
        HipError::check(unsafe { ffi::emel_memcpy_htod(self.ptr.cast(), data.as_ptr().cast(), bytes, stream.as_raw()) })?;
        stream.synchronize()
    }

    /// Copies the start of the buffer into `out` and waits for the copy, after
    /// every launch enqueued before it on `stream`.
    ///
    /// # Errors
    /// `EMEL_ERR_INVALID_ARGUMENT` when `out` is longer than the buffer, else
    /// the library status of the copy or the wait.
    pub fn copy_to_host(&self, out: &mut [T], stream: &Stream) -> Result<(), HipError> {
        if out.len() > self.len {
            return Err(HipError(ffi::EMEL_ERR_INVALID_ARGUMENT));
        }
        if out.is_empty() {
            return Ok(());
        }
        let bytes = size_of_val(out) as u64;
        // SAFETY: both ranges hold `bytes` bytes; the wait below completes the
        // write into `out` before it is released.
        HipError::check(unsafe { ffi::emel_memcpy_dtoh(out.as_mut_ptr().cast(), self.ptr.cast(), bytes, stream.as_raw()) })?;
        stream.synchronize()
    }

    /// Number of values.
    #[must_use]
    pub const fn len(&self) -> usize {
        self.len
    }

    /// Whether the buffer holds no values.
    #[must_use]
    pub const fn is_empty(&self) -> bool {
        self.len == 0
    }

    /// Size in bytes.
    #[must_use]
    pub const fn byte_len(&self) -> usize {
        self.len * size_of::<T>()
    }

    /// The device address.
    #[must_use]
    pub const fn as_ptr(&self) -> *const T {
        self.ptr
    }

    /// The device address, writable.
    #[must_use]
    pub const fn as_mut_ptr(&mut self) -> *mut T {
        self.ptr
    }

    /// Enqueues a bit copy of `src` into the start of this buffer with one
    /// streaming shape (`ffi::EMEL_COPY_*`): a measurement reference for
    /// what a plain stream achieves at this size.
    ///
    /// # Errors
    /// `EMEL_ERR_INVALID_ARGUMENT` when `src` is longer than the buffer, the
    /// byte count is not a multiple of 16 or the shape is unknown, else the
    /// library status of the launch.
    pub fn stream_copy_from(&mut self, src: &Self, shape: u32, stream: &Stream) -> Result<(), HipError> {
        if src.len > self.len {
            return Err(HipError(ffi::EMEL_ERR_INVALID_ARGUMENT));
        }
        // SAFETY: both device ranges hold src.byte_len() bytes and stay
        // allocated while `self` and `src` are borrowed; the library checks
        // alignment and the shape.
        HipError::check(unsafe {
            ffi::emel_stream_copy(src.ptr.cast(), self.ptr.cast(), src.byte_len() as u64, shape, stream.as_raw())
        })
    }
}

impl<T: Copy> Drop for DeviceBuffer<T> {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            // SAFETY: allocated by emel_malloc and freed once.
            let _ = unsafe { ffi::emel_free(self.ptr.cast()) };
        }
    }
}
