"""ctypes binding of include/emel_hip.h (libemel_hip.so).

The library is loaded from this package directory.  There is no fallback:
if libemel_hip.so is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import enum
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libemel_hip.so"


class Status(enum.IntEnum):
    """emel_status: one value per variant of the reference's typed errors."""

    OK = 0
    INVALID_VIEW = 1
    SHAPE_MISMATCH = 2
    INVALID_PARAMETERS = 3
    UNEXPECTED_EVENT = 4
    INTERNAL = 5
    KERNEL_UNAVAILABLE = 6
    DEVICE = 7
    INVALID_ARGUMENT = 8
    INVALID_SHAPE = 9
    UNSUPPORTED_OPERATION = 10


class DType(enum.IntEnum):
    """Wire dtype codes (DType::from_code, tensor_view.rs:111-158)."""

    F32 = 0
    F16 = 1
    I32 = 26


class UnarySubOp(enum.IntEnum):
    """UnarySubOp wire codes (unary.rs:101-146)."""

    ABS = 0
    SGN = 1
    NEG = 2
    STEP = 3
    TANH = 4
    ELU = 5
    RELU = 6
    SIGMOID = 7
    GELU = 8
    GELU_QUICK = 9
    SILU = 10
    HARDSWISH = 11
    HARDSIGMOID = 12
    EXP = 13


class GluSubOp(enum.IntEnum):
    """GluSubOp wire codes (glu.rs:22-37)."""

    REGLU = 0
    GEGLU = 1
    SWIGLU = 2
    SWIGLU_OAI = 3
    GEGLU_ERF = 4
    GEGLU_QUICK = 5


class BinaryOp(enum.IntEnum):
    ADD = 0
    SUB = 1
    MUL = 2
    DIV = 3


class CView(ctypes.Structure):
    """emel_tensor_view / emel_tensor_view_mut (identical layouts)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("data_bytes", ctypes.c_uint64),
        ("dtype", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("ne", ctypes.c_uint64 * 4),
        ("nb", ctypes.c_uint64 * 4),
    ]


_V = ctypes.POINTER(CView)
_S = ctypes.c_void_p
_ST = ctypes.c_int

# name -> argtypes; every op returns emel_status
SIGNATURES = {
    "emel_op_add": [_V, _V, _V, _S],
    "emel_op_sub": [_V, _V, _V, _S],
    "emel_op_mul": [_V, _V, _V, _S],
    "emel_op_div": [_V, _V, _V, _S],
    "emel_op_add_broadcast_row": [_V, _V, _V, _S],
    "emel_op_mul_broadcast_row": [_V, _V, _V, _S],
    "emel_op_binary_broadcast": [ctypes.c_int, _V, _V, _V, _S],
    "emel_op_unary": [ctypes.c_int, _V, _V, _S],
    "emel_op_silu": [_V, _V, _S],
    "emel_op_gelu": [_V, _V, _S],
    "emel_op_swiglu": [_V, _V, _V, _S],
    "emel_op_glu": [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, _S],
    "emel_slice_dup": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, _S],
    "emel_slice_sqr": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, _S],
    "emel_slice_sqrt": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, _S],
    **{f"emel_slice_{op}": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                            ctypes.c_uint64, _S] for op in ("add", "sub", "mul", "div")},
    "emel_op_sqr": [_V, _V, _S],
    "emel_op_sqrt": [_V, _V, _S],
    "emel_op_scale": [_V, _V, ctypes.c_float, _S],
    "emel_op_rms_norm": [_V, _V, ctypes.c_float, _S],
    "emel_op_rms_norm_mul": [_V, _V, _V, ctypes.c_float, _S],
    "emel_op_norm": [_V, _V, ctypes.c_float, _S],
    "emel_op_soft_max": [_V, _V, _S],
    "emel_op_soft_max_ext": [_V, _V, ctypes.c_float, _V, _S],
    "emel_op_sum_rows": [_V, _V, _S],
    "emel_op_sum": [_V, _V, _S],
    "emel_op_mean": [_V, _V, _S],
    "emel_op_argmax": [_V, _V, _S],
    "emel_op_argmax_rows": [_V, _V, _S],
    "emel_validate_view": [_V, ctypes.c_int32],
    "emel_validate_normalization_view": [_V],
    "emel_device_count": [ctypes.POINTER(ctypes.c_int32)],
    "emel_set_device": [ctypes.c_int32],
    "emel_malloc": [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint64],
    "emel_free": [ctypes.c_void_p],
    "emel_memcpy_htod": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, _S],
    "emel_memcpy_dtoh": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, _S],
    "emel_stream_create": [ctypes.POINTER(ctypes.c_void_p)],
    "emel_stream_destroy": [_S],
    "emel_stream_synchronize": [_S],
    "emel_release_workspaces": [],
}

_lib = None


def _share_torch_hip_runtime() -> None:
    """A process must hold one HIP runtime.  torch's libtorch_hip.so loads its
    bundled libamdhip64.so by file name; libemel_hip.so asks for the soname
    libamdhip64.so.7, which the bundled runtime also carries.  Importing torch
    first makes libemel_hip.so bind to torch's runtime, so both see the same
    devices and memory.  (Without torch, the system ROCm runtime is used.)"""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load() -> ctypes.CDLL:
    """Loads libemel_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        _share_torch_hip_runtime()
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _ST
        lib.emel_abi_version.restype = ctypes.c_uint32
        lib.emel_abi_version.argtypes = []
        lib.emel_status_string.restype = ctypes.c_char_p
        lib.emel_status_string.argtypes = [ctypes.c_int]
        lib.emel_last_error.restype = ctypes.c_char_p
        lib.emel_last_error.argtypes = []
        _lib = lib
    return _lib


def last_error() -> str:
    return load().emel_last_error().decode()


def device_count() -> int:
    n = ctypes.c_int32(0)
    load().emel_device_count(ctypes.byref(n))
    return int(n.value)
