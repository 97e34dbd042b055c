//! MI355X (gfx950) kernels behind emel's kernel-event API.
//!
//! [`HipKernel::process_event`] accepts the events of
//! `emel_kernels::any::event` re-expressed over device memory and returns
//! the same result types as the CPU actor's `Kernel::process_event`
//! (crates/emel-kernels/src/any/actor.rs:936-943), so a caller can run an
//! event on either and compare.  The device work is done by `libemel_hip`
//! (hand-written HIP kernels behind the C ABI of `include/emel_hip.h`);
//! this crate converts views and maps statuses, and leaves every guard to
//! the library.
//!
//! ```ignore
//! use emel_kernels::any::tensor_view::{DType, Layout};
//! use emel_kernels_hip::{DeviceBuffer, DeviceView, DeviceViewMut, HipKernel, event::OpSilu};
//!
//! let mut kernel = HipKernel::new()?;
//! let layout = Layout::contiguous(DType::F32, [4096, 32, 1, 1]).unwrap();
//! let x = DeviceBuffer::<f32>::from_host(&host_x, kernel.stream())?;
//! let mut y = DeviceBuffer::<f32>::new(x.len())?;
//! kernel.process_event(OpSilu::new(DeviceView::new(&x, layout), DeviceViewMut::new(&mut y, layout)))?;
//! y.copy_to_host(&mut host_y, kernel.stream())?; // waits for the launch
//! ```

#![allow(unsafe_code)] // an FFI crate: every unsafe block carries its SAFETY note

mod device;
pub mod event;
pub mod ffi;
pub mod graph;
mod kernel;
pub mod logits;
mod status;
mod view;

pub use device::{
    DeviceBuffer, HipError, Stream, abi_version, device_count, last_error, release_workspaces, set_device,
};
pub use kernel::{HipEvent, HipKernel};
pub use status::FromStatus;
pub use view::{DeviceIndexView, DeviceSlice, DeviceSliceMut, DeviceView, DeviceViewMut, IndexMemory};
