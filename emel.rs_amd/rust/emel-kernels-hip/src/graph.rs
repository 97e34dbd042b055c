//! The graph processor's kernel phase on the device: a `RunKernelFn`
//! (`fn(&ExecuteRequest, &mut i32) -> bool`,
//! crates/emel-graph/src/processor/sm.rs:159) that runs a [`HipStep`].

use emel_graph::{ExecuteRequest, ProcessorError, RunKernelFn};

use crate::kernel::HipKernel;

/// One graph step's device work: the kernel it runs on and a function that
/// enqueues the step's events.  `run` returns `Err(code)` with a
/// `ProcessorError` code (0 is read as `KernelFailed`) when an event fails.
#[derive(Debug)]
pub struct HipStep {
    /// The kernel (stream) the step's events are enqueued on.
    pub kernel: HipKernel,
    /// Enqueues the step's events.
    pub run: fn(&mut HipKernel, &ExecuteRequest) -> Result<(), i32>,
}

impl HipStep {
    /// The value to place in `ExecuteRequest::compute_ctx`.  The step must
    /// stay in place, and not be otherwise borrowed, while the processor
    /// dispatches the request.
    pub fn compute_ctx(&mut self) -> usize {
        core::ptr::from_mut(self) as usize
    }
}

/// Runs the [`HipStep`] at `request.compute_ctx` and waits for its launches,
/// so the next phase (`extract_outputs`) reads finished results, as after
/// the reference's synchronous kernel phase.  On failure `err` receives a
/// `ProcessorError` code: `InvalidRequest` for a null context, otherwise the
/// step's code or `KernelFailed`.
pub fn run_kernel(request: &ExecuteRequest, err: &mut i32) -> bool {
    if request.compute_ctx == 0 {
        *err = ProcessorError::InvalidRequest as i32;
        return false;
    }
    // SAFETY: compute_ctx came from HipStep::compute_ctx and the step is
    // live and exclusively ours for the duration of the dispatch.
    let step = unsafe { &mut *(request.compute_ctx as *mut HipStep) };
    let result = (step.run)(&mut step.kernel, request)
        .and_then(|()| step.kernel.synchronize().map_err(|_| ProcessorError::KernelFailed as i32));
    match result {
        Ok(()) => true,
        Err(code) => {
            *err = if code == 0 { ProcessorError::KernelFailed as i32 } else { code };
            false
        }
    }
}

/// [`run_kernel`] as the processor's callback type, for
/// `ExecuteRequest { run_kernel: Some(RUN_KERNEL), compute_ctx, .. }`.
pub const RUN_KERNEL: RunKernelFn = run_kernel;
