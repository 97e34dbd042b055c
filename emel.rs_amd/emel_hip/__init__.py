"""emel_hip: MI355X (gfx950) implementation of emel.rs's tensor-library hot
path -- elementwise, broadcast and row-reduction ops -- behind the C ABI in
include/emel_hip.h, with a Python mirror of emel-kernels' operator API.
"""
from .abi import BinaryOp, DType, GenericOp, GluSubOp, Status, UnarySubOp, device_count, last_error, load
from .generic import GenericEvent, GenericRequest, OpParams
from .get_rows import (IndexView, OpGetRows, OpGetRowsBf16, OpGetRowsF16, OpGetRowsF32Bytes, OpGetRowsQ4_0,
                       OpGetRowsQ4K, OpGetRowsQ8_0)
from .kernel import (
    DenseOpAdd,
    DenseOpDiv,
    DenseOpDup,
    DenseOpMul,
    DenseOpSqr,
    DenseOpSqrt,
    DenseOpSub,
    Kernel,
    OpAdd,
    OpAddBroadcastRow,
    OpArgmax,
    OpArgmaxRows,
    OpBinaryBroadcast,
    OpDiv,
    OpGelu,
    OpGlu,
    OpMean,
    OpMul,
    OpMulBroadcastRow,
    OpNorm,
    OpRmsNorm,
    OpRmsNormMul,
    OpScale,
    OpSilu,
    OpSoftMax,
    OpSoftMaxExt,
    OpSqr,
    OpSqrt,
    OpSub,
    OpSum,
    OpSumRows,
    OpSwiglu,
    OpUnary,
)
from .sampler import Build, SamplePreselected, Sampler, SampleTemperatureTopK, Validator
from .views import Layout, TensorView, TensorViewMut

__all__ = [
    "BinaryOp", "DType", "GenericOp", "GenericEvent", "GenericRequest", "OpParams", "GluSubOp", "Status", "UnarySubOp", "device_count", "last_error", "load",
    "Kernel", "Layout", "TensorView", "TensorViewMut",
    "OpAdd", "OpSub", "OpMul", "OpDiv", "OpAddBroadcastRow", "OpMulBroadcastRow", "OpBinaryBroadcast",
    "OpUnary", "OpSilu", "OpGelu", "OpGlu", "OpSwiglu", "OpScale", "OpRmsNorm", "OpRmsNormMul", "OpNorm",
    "OpSoftMax", "OpSoftMaxExt", "OpSumRows", "OpSum", "OpMean", "OpArgmax", "OpArgmaxRows",
    "OpSqr", "OpSqrt", "DenseOpDup", "DenseOpAdd", "DenseOpSub", "DenseOpMul", "DenseOpDiv", "DenseOpSqr",
    "DenseOpSqrt", "IndexView", "OpGetRows", "OpGetRowsF32Bytes", "OpGetRowsF16", "OpGetRowsBf16", "OpGetRowsQ4_0",
    "OpGetRowsQ8_0", "OpGetRowsQ4K", "Sampler", "SampleTemperatureTopK", "SamplePreselected", "Validator", "Build",
]
