//! Library statuses mapped onto the reference's per-family error enums.
//!
//! Each family maps the statuses its guards can produce to the variant of
//! the same name (the header documents one status per variant).  Statuses
//! no reference variant covers (a HIP runtime failure, no gfx950 device, a
//! call refused under stream capture, a NULL argument) map to `Internal`;
//! [`crate::HipKernel::last_status`] keeps the library status itself.

use emel_kernels::Error as KernelError;
use emel_kernels::any::event::{
    ActivationError, BinaryError, BroadcastError, DiagError, ElementwiseError, GetRowsError,
    GluError, GroupNormError, NormalizationError, ReductionError, UnaryError, UnsupportedOperation,
};
use emel_kernels::any::generic::KernelOperation;
use emel_kernels::any::power::PowerError;

use crate::ffi;

/// Conversion of a library status into a reference result.
pub trait FromStatus: Sized {
    /// `Ok(())` for `EMEL_OK`, else the matching error.
    ///
    /// # Errors
    /// Every status other than `EMEL_OK`.
    fn from_status(status: ffi::Status) -> Result<(), Self>;
}

// The four-variant families: InvalidView, ShapeMismatch, UnexpectedEvent,
// Internal (binary.rs:20-29, broadcast.rs:28-38, unary.rs:22-31,
// reductions.rs:21-30, activation.rs, power.rs:19-28), plus the extra
// variants a family has.
macro_rules! view_family {
    ($err:ident $(, $code:path => $variant:ident)*) => {
        impl FromStatus for $err {
            fn from_status(status: ffi::Status) -> Result<(), Self> {
                match status {
                    ffi::EMEL_OK => Ok(()),
                    ffi::EMEL_ERR_INVALID_VIEW => Err(Self::InvalidView),
                    ffi::EMEL_ERR_SHAPE_MISMATCH => Err(Self::ShapeMismatch),
                    ffi::EMEL_ERR_UNEXPECTED_EVENT => Err(Self::UnexpectedEvent),
                    $($code => Err(Self::$variant),)*
                    _ => Err(Self::Internal),
                }
            }
        }
    };
}

view_family!(BinaryError);
view_family!(BroadcastError);
view_family!(UnaryError);
view_family!(ReductionError);
view_family!(ActivationError);
view_family!(PowerError);
view_family!(NormalizationError, ffi::EMEL_ERR_INVALID_PARAMETERS => InvalidParameters);
view_family!(ElementwiseError, ffi::EMEL_ERR_INVALID_OFFSET => InvalidOffset);
view_family!(
    GroupNormError,
    ffi::EMEL_ERR_INVALID_PARAMETERS => InvalidParameters,
    ffi::EMEL_ERR_ZERO_NORM => ZeroNorm
);
view_family!(
    GetRowsError,
    ffi::EMEL_ERR_INDEX_OUT_OF_BOUNDS => IndexOutOfBounds,
    ffi::EMEL_ERR_UNSUPPORTED_SOURCE_STRIDE => UnsupportedSourceStride
);

// DiagError / GluError {InvalidShape, UnexpectedEvent, Internal}
// (diag.rs:18-40, glu.rs:40-63).
macro_rules! shape_family {
    ($err:ident) => {
        impl FromStatus for $err {
            fn from_status(status: ffi::Status) -> Result<(), Self> {
                match status {
                    ffi::EMEL_OK => Ok(()),
                    ffi::EMEL_ERR_INVALID_SHAPE => Err(Self::InvalidShape),
                    ffi::EMEL_ERR_UNEXPECTED_EVENT => Err(Self::UnexpectedEvent),
                    _ => Err(Self::Internal),
                }
            }
        }
    };
}

shape_family!(DiagError);
shape_family!(GluError);

/// The root `Error` (actor.rs:88-101) for the dense slice events and the
/// generic envelope.  `EMEL_ERR_UNSUPPORTED_OPERATION` carries the
/// operation the request named, which the caller supplies.
pub(crate) fn root_error(status: ffi::Status, operation: Option<KernelOperation>) -> Result<(), KernelError> {
    match status {
        ffi::EMEL_OK => Ok(()),
        ffi::EMEL_ERR_INVALID_SHAPE => Err(KernelError::InvalidShape),
        ffi::EMEL_ERR_UNEXPECTED_EVENT => Err(KernelError::UnexpectedEvent),
        ffi::EMEL_ERR_UNSUPPORTED_OPERATION => Err(KernelError::UnsupportedOperation(
            operation.map_or(UnsupportedOperation::MulMat, UnsupportedOperation::Generic),
        )),
        _ => Err(KernelError::Internal),
    }
}

impl FromStatus for KernelError {
    fn from_status(status: ffi::Status) -> Result<(), Self> {
        root_error(status, None)
    }
}
