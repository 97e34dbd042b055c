"""Operator events and the Kernel actor, mirroring emel-kernels' portable router.

    kernel = Kernel()
    status = kernel.process_event(OpAdd(TensorView(a, lay), TensorView(b, lay),
                                        TensorViewMut(out, lay)))
    assert status == Status.OK

Each event class carries the constructor arguments of the reference event of
the same name (cited per class) and maps onto one C-ABI entry point.
`Kernel.process_event` dispatches on the kernel's HIP stream and, like the
reference's run-to-completion actors (actor.rs:936-943), waits for the work
to finish unless the kernel was created with `synchronous=False`.  Rejected
requests return the error status without touching dst.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from .abi import BinaryOp, Status, UnarySubOp, load
from .views import TensorView, TensorViewMut


def _p(view):
    return None if view is None else ctypes.byref(view.c())


@dataclass
class OpAdd:
    """binary::OpAdd::new(lhs, rhs, output) (binary.rs:47-81)."""

    lhs: TensorView
    rhs: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_add(_p(self.lhs), _p(self.rhs), _p(self.output), s)


@dataclass
class OpSub:
    """binary::OpSub::new(lhs, rhs, output) (binary.rs:47-81)."""

    lhs: TensorView
    rhs: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_sub(_p(self.lhs), _p(self.rhs), _p(self.output), s)


@dataclass
class OpMul:
    """binary::OpMul::new(lhs, rhs, output) (binary.rs:47-81)."""

    lhs: TensorView
    rhs: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_mul(_p(self.lhs), _p(self.rhs), _p(self.output), s)


@dataclass
class OpDiv:
    """binary::OpDiv::new(lhs, rhs, output) (binary.rs:47-81)."""

    lhs: TensorView
    rhs: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_div(_p(self.lhs), _p(self.rhs), _p(self.output), s)


@dataclass
class OpAddBroadcastRow:
    """broadcast::OpAddBroadcastRow::new(src0, src1, dst) (broadcast.rs:53-66)."""

    src0: TensorView
    src1: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_add_broadcast_row(_p(self.src0), _p(self.src1), _p(self.dst), s)


@dataclass
class OpMulBroadcastRow:
    """broadcast::OpMulBroadcastRow::new(src0, src1, dst) (broadcast.rs:68-84)."""

    src0: TensorView
    src1: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_mul_broadcast_row(_p(self.src0), _p(self.src1), _p(self.dst), s)


@dataclass
class OpBinaryBroadcast:
    """OpRepeat(src1 -> dst.ne) then the equal-count binary op (generic.rs:1641-1665)."""

    op: BinaryOp
    src0: TensorView
    src1: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_binary_broadcast(int(self.op), _p(self.src0), _p(self.src1), _p(self.dst), s)


@dataclass
class OpUnary:
    """unary::OpUnary::new(subop, input, output) (unary.rs:150-172)."""

    subop: UnarySubOp
    input: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_unary(int(self.subop), _p(self.input), _p(self.output), s)


@dataclass
class OpSilu:
    """unary::OpSilu::new(input, output) (unary.rs:82)."""

    input: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_silu(_p(self.input), _p(self.output), s)


@dataclass
class OpUnaryEvent:
    """One of the 21 typed unary events (unary.rs:72-92), keyed by the
    UnarySubOp code of its formula; the named classes below build it."""

    event: int
    input: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_unary_event(int(self.event), _p(self.input), _p(self.output), s)


def _typed_unary(name, code):
    def make(input, output):
        return OpUnaryEvent(code, input, output)
    make.__name__ = name
    make.__doc__ = f"unary::{name}::new(input, output) (unary.rs:72-92): UnarySubOp {code.name}."
    return make


OpAbs = _typed_unary("OpAbs", UnarySubOp.ABS)
OpSgn = _typed_unary("OpSgn", UnarySubOp.SGN)
OpNeg = _typed_unary("OpNeg", UnarySubOp.NEG)
OpStep = _typed_unary("OpStep", UnarySubOp.STEP)
OpTanh = _typed_unary("OpTanh", UnarySubOp.TANH)
OpElu = _typed_unary("OpElu", UnarySubOp.ELU)
OpRelu = _typed_unary("OpRelu", UnarySubOp.RELU)
OpSigmoid = _typed_unary("OpSigmoid", UnarySubOp.SIGMOID)
OpGeluQuick = _typed_unary("OpGeluQuick", UnarySubOp.GELU_QUICK)
OpHardswish = _typed_unary("OpHardswish", UnarySubOp.HARDSWISH)
OpHardsigmoid = _typed_unary("OpHardsigmoid", UnarySubOp.HARDSIGMOID)
OpExp = _typed_unary("OpExp", UnarySubOp.EXP)
OpExpm1 = _typed_unary("OpExpm1", UnarySubOp.EXPM1)
OpSoftplus = _typed_unary("OpSoftplus", UnarySubOp.SOFTPLUS)
OpGeluErf = _typed_unary("OpGeluErf", UnarySubOp.GELU_ERF)
OpFloor = _typed_unary("OpFloor", UnarySubOp.FLOOR)
OpCeil = _typed_unary("OpCeil", UnarySubOp.CEIL)
OpRound = _typed_unary("OpRound", UnarySubOp.ROUND)
OpTrunc = _typed_unary("OpTrunc", UnarySubOp.TRUNC)


@dataclass
class OpLog:
    """reductions::OpLog::new(src, dst) (reductions.rs:45-58, :640-648)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_log(_p(self.src), _p(self.dst), s)


@dataclass
class OpSin:
    """reductions::OpSin::new(src, dst) (reductions.rs:60-73, :650-658)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_sin(_p(self.src), _p(self.dst), s)


@dataclass
class OpCos:
    """reductions::OpCos::new(src, dst) (reductions.rs:75-88, :660-668)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_cos(_p(self.src), _p(self.dst), s)


@dataclass
class OpGelu:
    """unary::OpGelu::new(input, output) (unary.rs:80)."""

    input: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_gelu(_p(self.input), _p(self.output), s)


@dataclass
class OpSwiglu:
    """OpSilu(gate) then OpMul by up, fused (unary.rs:595-600, binary.rs:411-424)."""

    gate: TensorView
    up: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_swiglu(_p(self.gate), _p(self.up), _p(self.output), s)


@dataclass
class OpGlu:
    """glu::OpGlu::new(input, output, subop) (glu.rs:69-92): input is a dense
    f32 slice [values | gates] of 2n floats, output n floats.  `input` and
    `output` are device tensors (or raw pointers, with the lengths given)."""

    input: object
    output: object
    subop: int
    input_len: int | None = None
    output_len: int | None = None

    def _call(self, lib, s):
        def ptr_len(t, n):
            if isinstance(t, int):
                return t, n
            return int(t.data_ptr()), (t.numel() if n is None else n)

        ip, il = ptr_len(self.input, self.input_len)
        op, ol = ptr_len(self.output, self.output_len)
        return lib.emel_op_glu(int(self.subop), ip, il, op, ol, s)


def _slice(t, n=None):
    """(device pointer, length in floats) of a tensor or raw pointer."""
    if isinstance(t, int):
        if n is None:
            raise ValueError("a raw pointer needs its length")
        return t, n
    return int(t.data_ptr()), (t.numel() if n is None else n)


@dataclass
class DenseOpDup:
    """event::OpDup::new(input, output) (event.rs:133-165): copy a slice."""

    input: object
    output: object
    input_len: int | None = None
    output_len: int | None = None

    def _call(self, lib, s):
        ip, il = _slice(self.input, self.input_len)
        op, ol = _slice(self.output, self.output_len)
        return lib.emel_slice_dup(ip, il, op, ol, s)


@dataclass
class _DenseBinary:
    lhs: object
    rhs: object
    output: object
    lhs_len: int | None = None
    rhs_len: int | None = None
    output_len: int | None = None
    _fn = ""

    def _call(self, lib, s):
        lp, ll = _slice(self.lhs, self.lhs_len)
        rp, rl = _slice(self.rhs, self.rhs_len)
        op, ol = _slice(self.output, self.output_len)
        return getattr(lib, self._fn)(lp, ll, rp, rl, op, ol, s)


class DenseOpAdd(_DenseBinary):
    """event::OpAdd::new(lhs, rhs, output) (event.rs:167-208)."""
    _fn = "emel_slice_add"


class DenseOpSub(_DenseBinary):
    """event::OpSub (event.rs:210-257)."""
    _fn = "emel_slice_sub"


class DenseOpMul(_DenseBinary):
    """event::OpMul (event.rs:210-258)."""
    _fn = "emel_slice_mul"


class DenseOpDiv(_DenseBinary):
    """event::OpDiv (event.rs:210-259)."""
    _fn = "emel_slice_div"


@dataclass
class _DenseUnary:
    input: object
    output: object
    input_len: int | None = None
    output_len: int | None = None
    _fn = ""

    def _call(self, lib, s):
        ip, il = _slice(self.input, self.input_len)
        op, ol = _slice(self.output, self.output_len)
        return getattr(lib, self._fn)(ip, il, op, ol, s)


class DenseOpSqr(_DenseUnary):
    """event::OpSqr::new(input, output) (event.rs:523-567)."""
    _fn = "emel_slice_sqr"


class DenseOpSqrt(_DenseUnary):
    """event::OpSqrt::new(input, output) (event.rs:523-568)."""
    _fn = "emel_slice_sqrt"


@dataclass
class OpSqr:
    """power::OpSqr::new(input, output) (power.rs:46-58)."""

    input: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_sqr(_p(self.input), _p(self.output), s)


@dataclass
class OpSqrt:
    """power::OpSqrt::new(input, output) (power.rs:60-73)."""

    input: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_sqrt(_p(self.input), _p(self.output), s)


@dataclass
class OpScale:
    """activation::OpScale::new(input, output, scale) (activation.rs:58-72)."""

    input: TensorView
    output: TensorViewMut
    scale: float

    def _call(self, lib, s):
        return lib.emel_op_scale(_p(self.input), _p(self.output), float(self.scale), s)


@dataclass
class OpRmsNorm:
    """normalization::OpRmsNorm::new(input, output, epsilon) (normalization.rs:80-96)."""

    input: TensorView
    output: TensorViewMut
    epsilon: float

    def _call(self, lib, s):
        return lib.emel_op_rms_norm(_p(self.input), _p(self.output), float(self.epsilon), s)


@dataclass
class OpRmsNormMul:
    """OpRmsNorm then OpMulBroadcastRow by a weight row, fused."""

    input: TensorView
    weight: TensorView
    output: TensorViewMut
    epsilon: float

    def _call(self, lib, s):
        return lib.emel_op_rms_norm_mul(_p(self.input), _p(self.weight), _p(self.output), float(self.epsilon), s)


@dataclass
class OpNorm:
    """normalization::OpNorm::new(input, output, epsilon) (normalization.rs:58-74)."""

    input: TensorView
    output: TensorViewMut
    epsilon: float

    def _call(self, lib, s):
        return lib.emel_op_norm(_p(self.input), _p(self.output), float(self.epsilon), s)


@dataclass
class OpSoftMax:
    """reductions::OpSoftMax::new(src, dst) (reductions.rs:152-163)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_soft_max(_p(self.src), _p(self.dst), s)


@dataclass
class OpSoftMaxExt:
    """OpScale -> OpAdd(f16 mask) -> OpSoftMax per (ne2, ne3) slice, fused."""

    src: TensorView
    mask: TensorView | None
    scale: float
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_soft_max_ext(_p(self.src), _p(self.mask), float(self.scale), _p(self.dst), s)


@dataclass
class OpSumRows:
    """reductions::OpSumRows::new(src, dst) (reductions.rs:107-118)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_sum_rows(_p(self.src), _p(self.dst), s)


@dataclass
class OpSum:
    """reductions::OpSum::new(src, dst) (reductions.rs:88-103)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_sum(_p(self.src), _p(self.dst), s)


@dataclass
class OpMean:
    """reductions::OpMean::new(src, dst) (reductions.rs:120-133)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_mean(_p(self.src), _p(self.dst), s)


@dataclass
class OpArgmax:
    """reductions::OpArgmax::new(src, dst) (reductions.rs:137-148)."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_argmax(_p(self.src), _p(self.dst), s)


@dataclass
class OpArgmaxRows:
    """One OpArgmax per row view, i32 indices."""

    src: TensorView
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_argmax_rows(_p(self.src), _p(self.dst), s)


class Kernel:
    """Single-writer actor over one HIP stream (Kernel, actor.rs:905-949)."""

    def __init__(self, stream: int | None = None, synchronous: bool = True):
        self._lib = load()
        self.stream = stream  # hipStream_t as an int, or None for the null stream
        self.synchronous = synchronous

    def process_event(self, event) -> Status:
        status = Status(event._call(self._lib, self.stream))
        if status == Status.OK and self.synchronous:
            sync = Status(self._lib.emel_stream_synchronize(self.stream))
            if sync != Status.OK:
                return sync
        return status


# ---- typed events of activation.rs, elementwise.rs, diag.rs, group_norm.rs ----

@dataclass
class OpClamp:
    """activation::OpClamp::new(input, output, min, max) (activation.rs:78-96)."""

    input: TensorView
    output: TensorViewMut
    min: float
    max: float

    def _call(self, lib, s):
        return lib.emel_op_clamp(_p(self.input), _p(self.output), self.min, self.max, s)


@dataclass
class OpLeakyRelu:
    """activation::OpLeakyRelu::new(input, output, negative_slope) (activation.rs:118-140)."""

    input: TensorView
    output: TensorViewMut
    negative_slope: float

    def _call(self, lib, s):
        return lib.emel_op_leaky_relu(_p(self.input), _p(self.output), self.negative_slope, s)


@dataclass
class OpSiluBack:
    """activation::OpSiluBack::new(input, gradient, output) (activation.rs:98-116)."""

    input: TensorView
    gradient: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_silu_back(_p(self.input), _p(self.gradient), _p(self.output), s)


@dataclass
class OpAdd1:
    """elementwise::OpAdd1::new(src, scalar, dst) (elementwise.rs:51-62)."""

    src: TensorView
    scalar: float
    dst: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_add1(_p(self.src), self.scalar, _p(self.dst), s)


@dataclass
class OpAcc:
    """elementwise::OpAcc::new(base, update, dst, offset) (elementwise.rs:64-80)."""

    base: TensorView
    update: TensorView
    dst: TensorViewMut
    offset: int

    def _call(self, lib, s):
        return lib.emel_op_acc(_p(self.base), _p(self.update), _p(self.dst), self.offset, s)


@dataclass
class OpDiag:
    """diag::OpDiag::new(input, output) (diag.rs:38-65): device tensors as slices."""

    input: object
    output: object
    input_len: int | None = None
    output_len: int | None = None

    def _call(self, lib, s):
        ip, il = _slice(self.input, self.input_len)
        op, ol = _slice(self.output, self.output_len)
        return lib.emel_op_diag(ip, il, op, ol, s)


@dataclass
class OpDiagMaskInf:
    """diag::OpDiagMaskInf::new(input, output, n_past) (diag.rs:67-85)."""

    input: object
    output: object
    n_past: int
    input_len: int | None = None
    output_len: int | None = None
    _fn = "emel_op_diag_mask_inf"

    def _call(self, lib, s):
        ip, il = _slice(self.input, self.input_len)
        op, ol = _slice(self.output, self.output_len)
        return getattr(lib, self._fn)(ip, il, op, ol, self.n_past, s)


@dataclass
class OpDiagMaskZero(OpDiagMaskInf):
    """diag::OpDiagMaskZero::new(input, output, n_past) (diag.rs:87-105)."""

    _fn = "emel_op_diag_mask_zero"


@dataclass
class OpGroupNorm:
    """group_norm::OpGroupNorm::new(input, output, groups, epsilon) (group_norm.rs:49-66)."""

    input: TensorView
    output: TensorViewMut
    groups: int
    epsilon: float

    def _call(self, lib, s):
        return lib.emel_op_group_norm(_p(self.input), _p(self.output), self.groups, self.epsilon, s)


@dataclass
class OpL2Norm:
    """group_norm::OpL2Norm::new(input, output) (group_norm.rs:68-78)."""

    input: TensorView
    output: TensorViewMut

    def _call(self, lib, s):
        return lib.emel_op_l2_norm(_p(self.input), _p(self.output), s)
