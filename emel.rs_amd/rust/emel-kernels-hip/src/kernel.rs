//! The device kernel actor: the reference's `Kernel::process_event`
//! (crates/emel-kernels/src/any/actor.rs:905-943) over HIP.

use crate::device::{HipError, Stream, abi_version};
use crate::ffi;

/// An event accepted by [`HipKernel`]; `Output` is the reference event's
/// result type (`BinaryResult`, `UnaryResult`, ...), or `Result<(),
/// HipError>` for the fused events the reference composes from several.
pub trait HipEvent: Sized {
    /// Result returned once the event's guards have run and its launches are
    /// enqueued.
    type Output;

    #[doc(hidden)]
    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output;
}

/// Dispatches kernel events to the MI355X library on one stream.
///
/// The reference actor returns after writing its output.  Here every guard
/// runs on the host before anything is enqueued, so the returned `Result`
/// is final when `process_event` returns, and the output is written when the
/// stream reaches the launches: read it after [`HipKernel::synchronize`] (or
/// a copy on the same stream), or set [`HipKernel::set_blocking`] to wait
/// inside every call as the reference does.
#[derive(Debug)]
pub struct HipKernel {
    stream: Stream,
    blocking: bool,
    last_status: ffi::Status,
}

impl HipKernel {
    /// A kernel on a new stream of the current device.
    ///
    /// # Errors
    /// `EMEL_ERR_KERNEL_UNAVAILABLE` when the loaded library's ABI version
    /// differs from this crate's or no gfx950 device is visible, else the
    /// status of the stream's creation.
    pub fn new() -> Result<Self, HipError> {
        Self::check_library()?;
        Ok(Self::on_stream(Stream::new()?))
    }

    /// A kernel that enqueues on `stream`.
    #[must_use]
    pub const fn on_stream(stream: Stream) -> Self {
        Self { stream, blocking: false, last_status: ffi::EMEL_OK }
    }

    fn check_library() -> Result<(), HipError> {
        if abi_version() != ffi::EMEL_HIP_ABI_VERSION {
            return Err(HipError(ffi::EMEL_ERR_KERNEL_UNAVAILABLE));
        }
        if crate::device::device_count()? == 0 {
            return Err(HipError(ffi::EMEL_ERR_KERNEL_UNAVAILABLE));
        }
        Ok(())
    }

    /// Dispatches one event (the reference's `process_event`).
    pub fn process_event<E: HipEvent>(&mut self, event: E) -> E::Output {
        event.dispatch(self)
    }

    /// When set, every event waits for its launches before returning.
    pub const fn set_blocking(&mut self, blocking: bool) {
        self.blocking = blocking;
    }

    /// The library status of the last event (kept when the typed error folds
    /// several statuses into `Internal`).
    #[must_use]
    pub const fn last_status(&self) -> ffi::Status {
        self.last_status
    }

    /// The stream the kernel enqueues on.
    #[must_use]
    pub const fn stream(&self) -> &Stream {
        &self.stream
    }

    /// Waits for every launch enqueued so far.
    ///
    /// # Errors
    /// The runtime status of a failed wait or kernel.
    pub fn synchronize(&self) -> Result<(), HipError> {
        self.stream.synchronize()
    }

    /// Runs one library call on the kernel's stream and records its status;
    /// in blocking mode a successful call is followed by a wait.
    pub(crate) fn call(&mut self, f: impl FnOnce(ffi::Stream) -> ffi::Status) -> ffi::Status {
        let mut status = f(self.stream.as_raw());
        if status == ffi::EMEL_OK && self.blocking {
            if let Err(HipError(wait)) = self.stream.synchronize() {
                status = wait;
            }
        }
        self.last_status = status;
        status
    }
}
