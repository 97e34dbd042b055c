//! Kernel events over device memory, named and constructed as in
//! `emel_kernels::any::event` (crates/emel-kernels/src/any/event.rs), each
//! returning the reference event's result type.
//!
//! `TensorView` / `TensorViewMut` operands become [`DeviceView`] /
//! [`DeviceViewMut`], `&[f32]` / `&mut [f32]` become [`DeviceSlice`] /
//! [`DeviceSliceMut`]; argument order and meaning are the reference's.

use emel_kernels::Error as KernelError;
use emel_kernels::any::event::{
    ActivationError, BinaryError, BroadcastError, DiagError, ElementwiseError, GetRowsError,
    GluError, GluSubOp, GroupNormError, KernelOperation, NormalizationError, ReductionError,
    UnaryError, UnarySubOp,
};

use crate::device::HipError;
use crate::ffi;
use crate::kernel::{HipEvent, HipKernel};
use crate::status::{FromStatus, root_error};
use crate::view::{DeviceIndexView, DeviceSlice, DeviceSliceMut, DeviceView, DeviceViewMut};

// ---- (input, output) tensor events ------------------------------------------

macro_rules! in_out_event {
    ($(#[$doc:meta])* $name:ident, $err:ty, |$i:ident, $o:ident, $s:ident| $call:expr) => {
        $(#[$doc])*
        #[derive(Debug)]
        pub struct $name<'a> {
            input: DeviceView<'a>,
            output: DeviceViewMut<'a>,
        }

        impl<'a> $name<'a> {
            /// Creates the event; validation occurs when it is dispatched.
            #[must_use]
            pub const fn new(input: DeviceView<'a>, output: DeviceViewMut<'a>) -> Self {
                Self { input, output }
            }
        }

        impl HipEvent for $name<'_> {
            type Output = Result<(), $err>;

            fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
                let $i = self.input.as_ffi();
                let $o = self.output.as_ffi();
                // SAFETY: both views describe live device memory for the
                // event's lifetime; the library checks every access against
                // data_bytes before launching.
                let status = kernel.call(|$s| unsafe { $call });
                <$err>::from_status(status)
            }
        }
    };
}

macro_rules! typed_unary {
    ($($(#[$doc:meta])* $name:ident = $code:path;)*) => {
        $(in_out_event!(
            $(#[$doc])* $name, UnaryError,
            |i, o, s| ffi::emel_op_unary_event($code, i, o, s)
        );)*
    };
}

typed_unary! {
    /// `OpAbs` (unary.rs): |x|.
    OpAbs = ffi::EMEL_UNARY_ABS;
    /// `OpSgn`: sign of x, 0 for zeros, NaN kept.
    OpSgn = ffi::EMEL_UNARY_SGN;
    /// `OpNeg`: -x.
    OpNeg = ffi::EMEL_UNARY_NEG;
    /// `OpStep`: 1 for x > 0, else 0.
    OpStep = ffi::EMEL_UNARY_STEP;
    /// `OpTanh`: glibc-exact tanhf.
    OpTanh = ffi::EMEL_UNARY_TANH;
    /// `OpElu`: x for x > 0, else expm1f(x).
    OpElu = ffi::EMEL_UNARY_ELU;
    /// `OpRelu`: f32::max(x, 0).
    OpRelu = ffi::EMEL_UNARY_RELU;
    /// `OpSigmoid`: 1 / (1 + expf(-x)).
    OpSigmoid = ffi::EMEL_UNARY_SIGMOID;
    /// `OpGeluQuick`: x * sigmoid(1.702 x).
    OpGeluQuick = ffi::EMEL_UNARY_GELU_QUICK;
    /// `OpHardswish`.
    OpHardswish = ffi::EMEL_UNARY_HARDSWISH;
    /// `OpHardsigmoid`.
    OpHardsigmoid = ffi::EMEL_UNARY_HARDSIGMOID;
    /// `OpExp`: glibc-exact expf.
    OpExp = ffi::EMEL_UNARY_EXP;
    /// `OpExpm1`: glibc-exact expm1f.
    OpExpm1 = ffi::EMEL_UNARY_EXPM1;
    /// `OpSoftplus`: log1pf(expf(x)).
    OpSoftplus = ffi::EMEL_UNARY_SOFTPLUS;
    /// `OpGeluErf`: the erf form of gelu.
    OpGeluErf = ffi::EMEL_UNARY_GELU_ERF;
    /// `OpFloor`.
    OpFloor = ffi::EMEL_UNARY_FLOOR;
    /// `OpCeil`.
    OpCeil = ffi::EMEL_UNARY_CEIL;
    /// `OpRound`: half away from zero.
    OpRound = ffi::EMEL_UNARY_ROUND;
    /// `OpTrunc`.
    OpTrunc = ffi::EMEL_UNARY_TRUNC;
}

in_out_event!(
    /// `OpSilu`: x / (1 + expf(-x)), glibc-exact expf.
    OpSilu, UnaryError, |i, o, s| ffi::emel_op_silu(i, o, s)
);
in_out_event!(
    /// `OpGelu`: the tanh approximation.
    OpGelu, UnaryError, |i, o, s| ffi::emel_op_gelu(i, o, s)
);
in_out_event!(
    /// `reductions::OpLog` (reductions.rs): glibc-exact logf per element.
    OpLog, ReductionError, |i, o, s| ffi::emel_op_log(i, o, s)
);
in_out_event!(
    /// `reductions::OpSin`: glibc-exact sinf per element.
    OpSin, ReductionError, |i, o, s| ffi::emel_op_sin(i, o, s)
);
in_out_event!(
    /// `reductions::OpCos`: glibc-exact cosf per element.
    OpCos, ReductionError, |i, o, s| ffi::emel_op_cos(i, o, s)
);
in_out_event!(
    /// `reductions::OpSoftMax` (reductions.rs:152-163): per-row soft_max.
    OpSoftMax, ReductionError, |i, o, s| ffi::emel_op_soft_max(i, o, s)
);
in_out_event!(
    /// `reductions::OpSumRows`: per-row f64-accumulated sum.
    OpSumRows, ReductionError, |i, o, s| ffi::emel_op_sum_rows(i, o, s)
);
in_out_event!(
    /// `reductions::OpSum`: whole-tensor sum to one f32.
    OpSum, ReductionError, |i, o, s| ffi::emel_op_sum(i, o, s)
);
in_out_event!(
    /// `reductions::OpMean`: per-row mean.
    OpMean, ReductionError, |i, o, s| ffi::emel_op_mean(i, o, s)
);
in_out_event!(
    /// `reductions::OpArgmax` (reductions.rs:137-148): whole-tensor index of
    /// the first maximum, as f32.
    OpArgmax, ReductionError, |i, o, s| ffi::emel_op_argmax(i, o, s)
);
in_out_event!(
    /// `group_norm::OpL2Norm` (group_norm.rs:92): reads the sum of squares
    /// back to the host for the ZeroNorm guard, so it waits and cannot be
    /// captured into a graph.
    OpL2Norm, GroupNormError, |i, o, s| ffi::emel_op_l2_norm(i, o, s)
);

/// View events of `power.rs` (`OpSqr`, `OpSqrt` over tensor views; the names
/// at the top of this module are the dense slice events, as in the
/// reference's `event` module).
pub mod power {
    use emel_kernels::any::power::PowerError;

    use super::{DeviceView, DeviceViewMut, FromStatus, HipEvent, HipKernel, ffi};

    in_out_event!(
        /// `power::OpSqr` (power.rs:48-58): x * x.
        OpSqr, PowerError, |i, o, s| ffi::emel_op_sqr(i, o, s)
    );
    in_out_event!(
        /// `power::OpSqrt` (power.rs:63-73): sqrtf(x).
        OpSqrt, PowerError, |i, o, s| ffi::emel_op_sqrt(i, o, s)
    );
}

/// `unary::OpUnary` (unary.rs:150-162): one of the eight subops the wire
/// envelope accepts (abs, neg, tanh, elu, relu, gelu, silu, exp); the others
/// are `UnaryError::UnexpectedEvent`, as in the reference.
#[derive(Debug)]
pub struct OpUnary<'a> {
    subop: UnarySubOp,
    input: DeviceView<'a>,
    output: DeviceViewMut<'a>,
}

impl<'a> OpUnary<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(subop: UnarySubOp, input: DeviceView<'a>, output: DeviceViewMut<'a>) -> Self {
        Self { subop, input, output }
    }
}

impl HipEvent for OpUnary<'_> {
    type Output = Result<(), UnaryError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, o, code) = (self.input.as_ffi(), self.output.as_ffi(), u32::from(self.subop as u8));
        // SAFETY: live device views, checked by the library.
        let status = kernel.call(|s| unsafe { ffi::emel_op_unary(code, i, o, s) });
        UnaryError::from_status(status)
    }
}

// ---- (a, b, output) tensor events ---------------------------------------------

macro_rules! two_in_event {
    ($(#[$doc:meta])* $name:ident($a:ident, $b:ident, $out:ident), $err:ty, $f:path) => {
        $(#[$doc])*
        #[derive(Debug)]
        pub struct $name<'a> {
            $a: DeviceView<'a>,
            $b: DeviceView<'a>,
            $out: DeviceViewMut<'a>,
        }

        impl<'a> $name<'a> {
            /// Creates the event; validation occurs when it is dispatched.
            #[must_use]
            pub const fn new($a: DeviceView<'a>, $b: DeviceView<'a>, $out: DeviceViewMut<'a>) -> Self {
                Self { $a, $b, $out }
            }
        }

        impl HipEvent for $name<'_> {
            type Output = Result<(), $err>;

            fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
                let (a, b, o) = (self.$a.as_ffi(), self.$b.as_ffi(), self.$out.as_ffi());
                // SAFETY: live device views, checked by the library.
                let status = kernel.call(|s| unsafe { $f(a, b, o, s) });
                <$err>::from_status(status)
            }
        }
    };
}

two_in_event!(
    /// `binary::OpAdd` (binary.rs:46-80): equal-count elementwise lhs + rhs.
    OpAddTensorView(lhs, rhs, output), BinaryError, ffi::emel_op_add
);
two_in_event!(
    /// `binary::OpSub`: equal-count lhs - rhs.
    OpSubTensorView(lhs, rhs, output), BinaryError, ffi::emel_op_sub
);
two_in_event!(
    /// `binary::OpMul`: equal-count lhs * rhs.
    OpMulTensorView(lhs, rhs, output), BinaryError, ffi::emel_op_mul
);
two_in_event!(
    /// `binary::OpDiv`: equal-count lhs / rhs.
    OpDivTensorView(lhs, rhs, output), BinaryError, ffi::emel_op_div
);
two_in_event!(
    /// `broadcast::OpAddBroadcastRow` (broadcast.rs:60-70): src0 + src1
    /// repeated over rows.
    OpAddBroadcastRow(src0, src1, dst), BroadcastError, ffi::emel_op_add_broadcast_row
);
two_in_event!(
    /// `broadcast::OpMulBroadcastRow` (broadcast.rs:77-87).
    OpMulBroadcastRow(src0, src1, dst), BroadcastError, ffi::emel_op_mul_broadcast_row
);
two_in_event!(
    /// `activation::OpSiluBack` (activation.rs:103-117).
    OpSiluBack(input, gradient, output), ActivationError, ffi::emel_op_silu_back
);

// ---- (input, output, parameters) tensor events --------------------------------

/// `activation::OpScale` (activation.rs:60-70): x * scale.
#[derive(Debug)]
pub struct OpScale<'a> {
    input: DeviceView<'a>,
    output: DeviceViewMut<'a>,
    scale: f32,
}

impl<'a> OpScale<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceView<'a>, output: DeviceViewMut<'a>, scale: f32) -> Self {
        Self { input, output, scale }
    }
}

impl HipEvent for OpScale<'_> {
    type Output = Result<(), ActivationError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, o, k) = (self.input.as_ffi(), self.output.as_ffi(), self.scale);
        // SAFETY: live device views, checked by the library.
        let status = kernel.call(|s| unsafe { ffi::emel_op_scale(i, o, k, s) });
        ActivationError::from_status(status)
    }
}

/// `activation::OpClamp` (activation.rs:81-92): `f32::clamp` order.
#[derive(Debug)]
pub struct OpClamp<'a> {
    input: DeviceView<'a>,
    output: DeviceViewMut<'a>,
    min: f32,
    max: f32,
}

impl<'a> OpClamp<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceView<'a>, output: DeviceViewMut<'a>, min: f32, max: f32) -> Self {
        Self { input, output, min, max }
    }
}

impl HipEvent for OpClamp<'_> {
    type Output = Result<(), ActivationError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, o, lo, hi) = (self.input.as_ffi(), self.output.as_ffi(), self.min, self.max);
        // SAFETY: live device views, checked by the library.
        let status = kernel.call(|s| unsafe { ffi::emel_op_clamp(i, o, lo, hi, s) });
        ActivationError::from_status(status)
    }
}

/// `activation::OpLeakyRelu` (activation.rs:126-141).
#[derive(Debug)]
pub struct OpLeakyRelu<'a> {
    input: DeviceView<'a>,
    output: DeviceViewMut<'a>,
    negative_slope: f32,
}

impl<'a> OpLeakyRelu<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceView<'a>, output: DeviceViewMut<'a>, negative_slope: f32) -> Self {
        Self { input, output, negative_slope }
    }
}

impl HipEvent for OpLeakyRelu<'_> {
    type Output = Result<(), ActivationError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, o, k) = (self.input.as_ffi(), self.output.as_ffi(), self.negative_slope);
        // SAFETY: live device views, checked by the library.
        let status = kernel.call(|s| unsafe { ffi::emel_op_leaky_relu(i, o, k, s) });
        ActivationError::from_status(status)
    }
}

macro_rules! epsilon_event {
    ($(#[$doc:meta])* $name:ident, $f:path) => {
        $(#[$doc])*
        #[derive(Debug)]
        pub struct $name<'a> {
            input: DeviceView<'a>,
            output: DeviceViewMut<'a>,
            epsilon: f32,
        }

        impl<'a> $name<'a> {
            /// Creates the event; validation occurs when it is dispatched.
            #[must_use]
            pub const fn new(input: DeviceView<'a>, output: DeviceViewMut<'a>, epsilon: f32) -> Self {
                Self { input, output, epsilon }
            }
        }

        impl HipEvent for $name<'_> {
            type Output = Result<(), NormalizationError>;

            fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
                let (i, o, e) = (self.input.as_ffi(), self.output.as_ffi(), self.epsilon);
                // SAFETY: live device views, checked by the library.
                let status = kernel.call(|s| unsafe { $f(i, o, e, s) });
                NormalizationError::from_status(status)
            }
        }
    };
}

epsilon_event!(
    /// `normalization::OpNorm` (normalization.rs:62-76): per-row mean and
    /// variance normalisation.
    OpNorm, ffi::emel_op_norm
);
epsilon_event!(
    /// `normalization::OpRmsNorm` (normalization.rs:80-96).
    OpRmsNorm, ffi::emel_op_rms_norm
);

/// `elementwise::OpAdd1` (elementwise.rs:53-64): src + scalar.
#[derive(Debug)]
pub struct OpAdd1<'a> {
    src: DeviceView<'a>,
    scalar: f32,
    dst: DeviceViewMut<'a>,
}

impl<'a> OpAdd1<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(src: DeviceView<'a>, scalar: f32, dst: DeviceViewMut<'a>) -> Self {
        Self { src, scalar, dst }
    }
}

impl HipEvent for OpAdd1<'_> {
    type Output = Result<(), ElementwiseError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, k, o) = (self.src.as_ffi(), self.scalar, self.dst.as_ffi());
        // SAFETY: live device views, checked by the library.
        let status = kernel.call(|s| unsafe { ffi::emel_op_add1(i, k, o, s) });
        ElementwiseError::from_status(status)
    }
}

/// `elementwise::OpAcc` (elementwise.rs:75-94): dst = base with update added
/// from element `offset` on.
#[derive(Debug)]
pub struct OpAcc<'a> {
    base: DeviceView<'a>,
    update: DeviceView<'a>,
    dst: DeviceViewMut<'a>,
    offset: usize,
}

impl<'a> OpAcc<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(base: DeviceView<'a>, update: DeviceView<'a>, dst: DeviceViewMut<'a>, offset: usize) -> Self {
        Self { base, update, dst, offset }
    }
}

impl HipEvent for OpAcc<'_> {
    type Output = Result<(), ElementwiseError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (b, u, o, off) = (self.base.as_ffi(), self.update.as_ffi(), self.dst.as_ffi(), self.offset as u64);
        // SAFETY: live device views, checked by the library.
        let status = kernel.call(|s| unsafe { ffi::emel_op_acc(b, u, o, off, s) });
        ElementwiseError::from_status(status)
    }
}

/// `group_norm::OpGroupNorm` (group_norm.rs:60-80).
#[derive(Debug)]
pub struct OpGroupNorm<'a> {
    input: DeviceView<'a>,
    output: DeviceViewMut<'a>,
    groups: usize,
    epsilon: f32,
}

impl<'a> OpGroupNorm<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceView<'a>, output: DeviceViewMut<'a>, groups: usize, epsilon: f32) -> Self {
        Self { input, output, groups, epsilon }
    }
}

impl HipEvent for OpGroupNorm<'_> {
    type Output = Result<(), GroupNormError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, o, g, e) = (self.input.as_ffi(), self.output.as_ffi(), self.groups as u64, self.epsilon);
        // SAFETY: live device views, checked by the library.
        let status = kernel.call(|s| unsafe { ffi::emel_op_group_norm(i, o, g, e, s) });
        GroupNormError::from_status(status)
    }
}

// ---- dense slice events (root Error) ------------------------------------------

/// `event::OpDup` (event.rs:133-165): copies one dense f32 run into another.
#[derive(Debug)]
pub struct OpDup<'a> {
    input: DeviceSlice<'a>,
    output: DeviceSliceMut<'a>,
}

impl<'a> OpDup<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceSlice<'a>, output: DeviceSliceMut<'a>) -> Self {
        Self { input, output }
    }
}

impl HipEvent for OpDup<'_> {
    type Output = Result<(), KernelError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, ni, o, no) = (self.input.ptr(), self.input.len() as u64, self.output.ptr(), self.output.len() as u64);
        // SAFETY: the slices address ni / no live device floats.
        let status = kernel.call(|s| unsafe { ffi::emel_slice_dup(i, ni, o, no, s) });
        root_error(status, None)
    }
}

macro_rules! slice_binary {
    ($(#[$doc:meta])* $name:ident, $f:path) => {
        $(#[$doc])*
        #[derive(Debug)]
        pub struct $name<'a> {
            lhs: DeviceSlice<'a>,
            rhs: DeviceSlice<'a>,
            output: DeviceSliceMut<'a>,
        }

        impl<'a> $name<'a> {
            /// Creates the event; validation occurs when it is dispatched.
            #[must_use]
            pub const fn new(lhs: DeviceSlice<'a>, rhs: DeviceSlice<'a>, output: DeviceSliceMut<'a>) -> Self {
                Self { lhs, rhs, output }
            }
        }

        impl HipEvent for $name<'_> {
            type Output = Result<(), KernelError>;

            fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
                let (a, na) = (self.lhs.ptr(), self.lhs.len() as u64);
                let (b, nb) = (self.rhs.ptr(), self.rhs.len() as u64);
                let (o, no) = (self.output.ptr(), self.output.len() as u64);
                // SAFETY: the slices address na / nb / no live device floats.
                let status = kernel.call(|s| unsafe { $f(a, na, b, nb, o, no, s) });
                root_error(status, None)
            }
        }
    };
}

slice_binary!(
    /// `event::OpAdd` (event.rs:168-205): dense equal-length lhs + rhs.
    OpAdd, ffi::emel_slice_add
);
slice_binary!(
    /// `event::OpSub` (event.rs:210-259).
    OpSub, ffi::emel_slice_sub
);
slice_binary!(
    /// `event::OpMul`.
    OpMul, ffi::emel_slice_mul
);
slice_binary!(
    /// `event::OpDiv`.
    OpDiv, ffi::emel_slice_div
);

macro_rules! slice_unary {
    ($(#[$doc:meta])* $name:ident, $f:path) => {
        $(#[$doc])*
        #[derive(Debug)]
        pub struct $name<'a> {
            input: DeviceSlice<'a>,
            output: DeviceSliceMut<'a>,
        }

        impl<'a> $name<'a> {
            /// Creates the event; validation occurs when it is dispatched.
            #[must_use]
            pub const fn new(input: DeviceSlice<'a>, output: DeviceSliceMut<'a>) -> Self {
                Self { input, output }
            }
        }

        impl HipEvent for $name<'_> {
            type Output = Result<(), KernelError>;

            fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
                let (i, ni) = (self.input.ptr(), self.input.len() as u64);
                let (o, no) = (self.output.ptr(), self.output.len() as u64);
                // SAFETY: the slices address ni / no live device floats.
                let status = kernel.call(|s| unsafe { $f(i, ni, o, no, s) });
                root_error(status, None)
            }
        }
    };
}

slice_unary!(
    /// `event::OpSqr` (event.rs:567): dense x * x.
    OpSqr, ffi::emel_slice_sqr
);
slice_unary!(
    /// `event::OpSqrt` (event.rs:568): dense sqrtf(x).
    OpSqrt, ffi::emel_slice_sqrt
);

/// `glu::OpGlu` (glu.rs:70-80): value/gate halves of each row of `input`.
#[derive(Debug)]
pub struct OpGlu<'a> {
    input: DeviceSlice<'a>,
    output: DeviceSliceMut<'a>,
    subop: GluSubOp,
}

impl<'a> OpGlu<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceSlice<'a>, output: DeviceSliceMut<'a>, subop: GluSubOp) -> Self {
        Self { input, output, subop }
    }
}

impl HipEvent for OpGlu<'_> {
    type Output = Result<(), GluError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let code = u32::from(self.subop as u8);
        let (i, ni) = (self.input.ptr(), self.input.len() as u64);
        let (o, no) = (self.output.ptr(), self.output.len() as u64);
        // SAFETY: the slices address ni / no live device floats.
        let status = kernel.call(|s| unsafe { ffi::emel_op_glu(code, i, ni, o, no, s) });
        GluError::from_status(status)
    }
}

/// `diag::OpDiag` (diag.rs:46-60): a vector to the diagonal of a square
/// matrix.
#[derive(Debug)]
pub struct OpDiag<'a> {
    input: DeviceSlice<'a>,
    output: DeviceSliceMut<'a>,
}

impl<'a> OpDiag<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceSlice<'a>, output: DeviceSliceMut<'a>) -> Self {
        Self { input, output }
    }
}

impl HipEvent for OpDiag<'_> {
    type Output = Result<(), DiagError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, ni) = (self.input.ptr(), self.input.len() as u64);
        let (o, no) = (self.output.ptr(), self.output.len() as u64);
        // SAFETY: the slices address ni / no live device floats.
        let status = kernel.call(|s| unsafe { ffi::emel_op_diag(i, ni, o, no, s) });
        DiagError::from_status(status)
    }
}

macro_rules! diag_mask {
    ($(#[$doc:meta])* $name:ident, $f:path) => {
        $(#[$doc])*
        #[derive(Debug)]
        pub struct $name<'a> {
            input: DeviceSlice<'a>,
            output: DeviceSliceMut<'a>,
            n_past: i32,
        }

        impl<'a> $name<'a> {
            /// Creates the event; validation occurs when it is dispatched.
            #[must_use]
            pub const fn new(input: DeviceSlice<'a>, output: DeviceSliceMut<'a>, n_past: i32) -> Self {
                Self { input, output, n_past }
            }
        }

        impl HipEvent for $name<'_> {
            type Output = Result<(), DiagError>;

            fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
                let (i, ni) = (self.input.ptr(), self.input.len() as u64);
                let (o, no) = (self.output.ptr(), self.output.len() as u64);
                let n_past = self.n_past;
                // SAFETY: the slices address ni / no live device floats.
                let status = kernel.call(|s| unsafe { $f(i, ni, o, no, n_past, s) });
                DiagError::from_status(status)
            }
        }
    };
}

diag_mask!(
    /// `diag::OpDiagMaskInf` (diag.rs:71-82): -inf above the diagonal shifted
    /// by n_past.
    OpDiagMaskInf, ffi::emel_op_diag_mask_inf
);
diag_mask!(
    /// `diag::OpDiagMaskZero` (diag.rs:91-102): zero above it.
    OpDiagMaskZero, ffi::emel_op_diag_mask_zero
);

// ---- row gathers ------------------------------------------------------------------

macro_rules! get_rows_event {
    ($(#[$doc:meta])* $name:ident, $f:path) => {
        $(#[$doc])*
        #[derive(Debug)]
        pub struct $name<'a> {
            source: DeviceView<'a>,
            indices: DeviceIndexView<'a>,
            destination: DeviceViewMut<'a>,
        }

        impl<'a> $name<'a> {
            /// Creates the event; validation occurs when it is dispatched.
            #[must_use]
            pub const fn new(source: DeviceView<'a>, indices: DeviceIndexView<'a>, destination: DeviceViewMut<'a>) -> Self {
                Self { source, indices, destination }
            }
        }

        impl HipEvent for $name<'_> {
            type Output = Result<(), GetRowsError>;

            fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
                let (src, idx, dst) = (self.source.as_ffi(), self.indices.as_ffi(), self.destination.as_ffi());
                // SAFETY: live views; the library checks the index span and
                // every index before the gather.
                let status = kernel.call(|s| unsafe { $f(src, idx, dst, s) });
                GetRowsError::from_status(status)
            }
        }
    };
}

get_rows_event!(
    /// `get_rows::OpGetRows` (get_rows.rs:500-515): F32 rows.
    OpGetRows, ffi::emel_op_get_rows
);
get_rows_event!(
    /// `get_rows::OpGetRowsF32Bytes` (get_rows.rs:240-255): F32 rows whose
    /// byte strides need not be multiples of 4.
    OpGetRowsF32Bytes, ffi::emel_op_get_rows_f32_bytes
);
get_rows_event!(
    /// `get_rows::OpGetRowsF16` (get_rows.rs:410-425).
    OpGetRowsF16, ffi::emel_op_get_rows_f16
);
get_rows_event!(
    /// `get_rows::OpGetRowsBf16` (get_rows.rs:394-405).
    OpGetRowsBf16, ffi::emel_op_get_rows_bf16
);
get_rows_event!(
    /// `get_rows::OpGetRowsQ4_0` (get_rows.rs:435-450).
    OpGetRowsQ4_0, ffi::emel_op_get_rows_q4_0
);
get_rows_event!(
    /// `get_rows::OpGetRowsQ8_0` (get_rows.rs:460-475).
    OpGetRowsQ8_0, ffi::emel_op_get_rows_q8_0
);
get_rows_event!(
    /// `get_rows::OpGetRowsQ4K` (get_rows.rs:485-500).
    OpGetRowsQ4K, ffi::emel_op_get_rows_q4_k
);

// ---- generic wire envelope --------------------------------------------------------

/// `generic::GenericEvent` (generic.rs:634-797): the pinned operation struct
/// for any of the 95 operation codes.
#[derive(Debug)]
pub struct GenericEvent<'a> {
    operation: KernelOperation,
    src: [Option<DeviceView<'a>>; 3],
    dst: Option<DeviceViewMut<'a>>,
    op_params: [u8; 64],
    op_params_size: u32,
    unary: u32,
    index_out: *mut i32,
}

impl<'a> GenericEvent<'a> {
    /// A request for `operation` (`GenericRequest::new`): up to three
    /// sources, a destination and the first `op_params.len()` (at most 64)
    /// parameter bytes; longer parameter blocks are truncated to 64 and the
    /// library reports the request as invalid.
    #[must_use]
    pub fn new(
        operation: KernelOperation,
        src: [Option<DeviceView<'a>>; 3],
        dst: Option<DeviceViewMut<'a>>,
        op_params: &[u8],
    ) -> Self {
        let mut params = [0_u8; 64];
        let n = op_params.len().min(64);
        params[..n].copy_from_slice(&op_params[..n]);
        let size = if op_params.len() > 64 { 65 } else { n as u32 };
        Self { operation, src, dst, op_params: params, op_params_size: size, unary: 0, index_out: core::ptr::null_mut() }
    }

    /// Sets the unary subop read by `KernelOperation::Unary`
    /// (`GenericRequest::with_unary`).
    #[must_use]
    pub const fn with_unary(mut self, subop: UnarySubOp) -> Self {
        self.unary = subop as u32;
        self
    }

    /// Sets the device address that receives `mul_mat_argmax`'s row
    /// (`GenericRequest::with_index_out`).
    ///
    /// # Safety
    /// `index_out` must address one writable i32 on the current device for
    /// as long as the launch runs.
    #[must_use]
    pub const unsafe fn with_index_out(mut self, index_out: *mut i32) -> Self {
        self.index_out = index_out;
        self
    }
}

impl HipEvent for GenericEvent<'_> {
    type Output = Result<(), KernelError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let src = |k: usize| self.src[k].as_ref().map_or(core::ptr::null(), |v| core::ptr::from_ref(v.as_ffi()));
        let request = ffi::EmelGenericRequest {
            operation: u32::from(self.operation as u8),
            unary_subop: self.unary,
            glu_subop: 0,
            pool_subop: 0,
            src0: src(0),
            src1: src(1),
            src2: src(2),
            dst: self.dst.as_ref().map_or(core::ptr::null(), |v| core::ptr::from_ref(v.as_ffi())),
            op_params: self.op_params,
            op_params_size: self.op_params_size,
            reserved: 0,
            index_out: self.index_out,
        };
        // SAFETY: the request and its views live across the call; the library
        // validates every view before launching.
        let status = kernel.call(|s| unsafe { ffi::emel_generic_dispatch(&raw const request, s) });
        root_error(status, Some(self.operation))
    }
}

// ---- fused events (no reference counterpart: reference compositions) ------------

/// Fused SwiGLU: `OpSilu(gate)` then equal-count `OpMulTensorView` by `up`,
/// both f32 roundings kept.
#[derive(Debug)]
pub struct OpSwiglu<'a> {
    gate: DeviceView<'a>,
    up: DeviceView<'a>,
    output: DeviceViewMut<'a>,
}

impl<'a> OpSwiglu<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(gate: DeviceView<'a>, up: DeviceView<'a>, output: DeviceViewMut<'a>) -> Self {
        Self { gate, up, output }
    }
}

impl HipEvent for OpSwiglu<'_> {
    type Output = Result<(), HipError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (g, u, o) = (self.gate.as_ffi(), self.up.as_ffi(), self.output.as_ffi());
        // SAFETY: live device views, checked by the library.
        HipError::check(kernel.call(|s| unsafe { ffi::emel_op_swiglu(g, u, o, s) }))
    }
}

/// Fused `OpRmsNorm` then `OpMulBroadcastRow` by `weight`.
#[derive(Debug)]
pub struct OpRmsNormMul<'a> {
    input: DeviceView<'a>,
    weight: DeviceView<'a>,
    output: DeviceViewMut<'a>,
    epsilon: f32,
}

impl<'a> OpRmsNormMul<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(input: DeviceView<'a>, weight: DeviceView<'a>, output: DeviceViewMut<'a>, epsilon: f32) -> Self {
        Self { input, weight, output, epsilon }
    }
}

impl HipEvent for OpRmsNormMul<'_> {
    type Output = Result<(), HipError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (i, w, o, e) = (self.input.as_ffi(), self.weight.as_ffi(), self.output.as_ffi(), self.epsilon);
        // SAFETY: live device views, checked by the library.
        HipError::check(kernel.call(|s| unsafe { ffi::emel_op_rms_norm_mul(i, w, o, e, s) }))
    }
}

/// Scaled, masked soft_max: `OpScale`, equal-count `OpAdd` of the f16 mask,
/// dense `OpSoftMax`, per (ne2, ne3) slice; `mask` may be absent.
#[derive(Debug)]
pub struct OpSoftMaxExt<'a> {
    src: DeviceView<'a>,
    mask: Option<DeviceView<'a>>,
    scale: f32,
    dst: DeviceViewMut<'a>,
}

impl<'a> OpSoftMaxExt<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(src: DeviceView<'a>, mask: Option<DeviceView<'a>>, scale: f32, dst: DeviceViewMut<'a>) -> Self {
        Self { src, mask, scale, dst }
    }
}

impl HipEvent for OpSoftMaxExt<'_> {
    type Output = Result<(), HipError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let m = self.mask.as_ref().map_or(core::ptr::null(), |v| core::ptr::from_ref(v.as_ffi()));
        let (x, k, o) = (self.src.as_ffi(), self.scale, self.dst.as_ffi());
        // SAFETY: live device views, checked by the library.
        HipError::check(kernel.call(|s| unsafe { ffi::emel_op_soft_max_ext(x, m, k, o, s) }))
    }
}

/// Row-broadcast binary op for any of add, sub, mul, div: src1's rows
/// repeat over src0's (the broadcast events generalised to four ops).
#[derive(Debug)]
pub struct OpBinaryBroadcast<'a> {
    op: u32,
    src0: DeviceView<'a>,
    src1: DeviceView<'a>,
    dst: DeviceViewMut<'a>,
}

impl<'a> OpBinaryBroadcast<'a> {
    /// `op` is one of `ffi::EMEL_BINARY_ADD` / `SUB` / `MUL` / `DIV`.
    #[must_use]
    pub const fn new(op: u32, src0: DeviceView<'a>, src1: DeviceView<'a>, dst: DeviceViewMut<'a>) -> Self {
        Self { op, src0, src1, dst }
    }
}

impl HipEvent for OpBinaryBroadcast<'_> {
    type Output = Result<(), HipError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (op, a, b, o) = (self.op, self.src0.as_ffi(), self.src1.as_ffi(), self.dst.as_ffi());
        // SAFETY: live device views, checked by the library.
        HipError::check(kernel.call(|s| unsafe { ffi::emel_op_binary_broadcast(op, a, b, o, s) }))
    }
}

/// One `OpArgmax` per row, to an I32 destination of shape [1, ne1, ne2, ne3].
#[derive(Debug)]
pub struct OpArgmaxRows<'a> {
    src: DeviceView<'a>,
    dst: DeviceViewMut<'a>,
    no_alloc: bool,
}

impl<'a> OpArgmaxRows<'a> {
    /// Creates the event; validation occurs when it is dispatched.
    #[must_use]
    pub const fn new(src: DeviceView<'a>, dst: DeviceViewMut<'a>) -> Self {
        Self { src, dst, no_alloc: false }
    }

    /// Uses the entry point that allocates nothing (a fixed per-device
    /// workspace; calls that overlap on one device race).
    #[must_use]
    pub const fn without_allocation(mut self) -> Self {
        self.no_alloc = true;
        self
    }
}

impl HipEvent for OpArgmaxRows<'_> {
    type Output = Result<(), HipError>;

    fn dispatch(self, kernel: &mut HipKernel) -> Self::Output {
        let (x, o) = (self.src.as_ffi(), self.dst.as_ffi());
        let f = if self.no_alloc { ffi::emel_op_argmax_rows_no_alloc } else { ffi::emel_op_argmax_rows };
        // SAFETY: live device views, checked by the library.
        HipError::check(kernel.call(|s| unsafe { f(x, o, s) }))
    }
}
