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
    INDEX_OUT_OF_BOUNDS = 11
    UNSUPPORTED_SOURCE_STRIDE = 12
    INVALID_REQUEST = 13
    STREAM_CAPTURE = 14
    INVALID_OFFSET = 15
    ZERO_NORM = 16


class DType(enum.IntEnum):
    """Wire dtype codes (DType::from_code, tensor_view.rs:111-158)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4_K = 12
    I32 = 26
    BF16 = 30


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
    EXPM1 = 14
    SOFTPLUS = 15
    GELU_ERF = 16
    XIELU = 17
    FLOOR = 18
    CEIL = 19
    ROUND = 20
    TRUNC = 21


class GluSubOp(enum.IntEnum):
    """GluSubOp wire codes (glu.rs:22-37)."""

    REGLU = 0
    GEGLU = 1
    SWIGLU = 2
    SWIGLU_OAI = 3
    GEGLU_ERF = 4
    GEGLU_QUICK = 5


class GenericOp(enum.IntEnum):
    """KernelOperation wire codes (generic.rs:24-337): the 95 entries of the
    pinned EMEL_KERNEL_OP_EVENT_LIST, in order."""

    DUP = 0
    ADD = 1
    ADD_ID = 2
    ADD1 = 3
    ACC = 4
    SUB = 5
    MUL = 6
    DIV = 7
    SQR = 8
    SQRT = 9
    LOG = 10
    SIN = 11
    COS = 12
    SUM = 13
    SUM_ROWS = 14
    CUMSUM = 15
    MEAN = 16
    ARGMAX = 17
    COUNT_EQUAL = 18
    REPEAT = 19
    REPEAT_BACK = 20
    CONCAT = 21
    SILU_BACK = 22
    NORM = 23
    RMS_NORM = 24
    RMS_NORM_BACK = 25
    GROUP_NORM = 26
    L2_NORM = 27
    MUL_MAT = 28
    MUL_MAT_ARGMAX = 29
    MUL_MAT_ID = 30
    OUT_PROD = 31
    SCALE = 32
    SET = 33
    CPY = 34
    CONT = 35
    RESHAPE = 36
    VIEW = 37
    PERMUTE = 38
    TRANSPOSE = 39
    GET_ROWS = 40
    GET_ROWS_BACK = 41
    SET_ROWS = 42
    DIAG = 43
    DIAG_MASK_INF = 44
    DIAG_MASK_ZERO = 45
    SOFT_MAX = 46
    SOFT_MAX_BACK = 47
    ROPE = 48
    ROPE_BACK = 49
    CLAMP = 50
    CONV_TRANSPOSE_1D = 51
    IM2COL = 52
    IM2COL_BACK = 53
    IM2COL_3D = 54
    CONV_2D = 55
    CONV_3D = 56
    CONV_2D_DW = 57
    CONV_TRANSPOSE_2D = 58
    POOL_1D = 59
    POOL_2D = 60
    POOL_2D_BACK = 61
    UPSCALE = 62
    PAD = 63
    PAD_REFLECT_1D = 64
    ROLL = 65
    ARANGE = 66
    TIMESTEP_EMBEDDING = 67
    ARGSORT = 68
    TOP_K = 69
    LEAKY_RELU = 70
    TRI = 71
    FILL = 72
    FLASH_ATTN_EXT = 73
    FLASH_ATTN_BACK = 74
    SSM_CONV = 75
    SSM_SCAN = 76
    WIN_PART = 77
    WIN_UNPART = 78
    GET_REL_POS = 79
    ADD_REL_POS = 80
    RWKV_WKV6 = 81
    GATED_LINEAR_ATTN = 82
    RWKV_WKV7 = 83
    SOLVE_TRI = 84
    UNARY = 85
    MAP_CUSTOM1 = 86
    MAP_CUSTOM2 = 87
    MAP_CUSTOM3 = 88
    CUSTOM = 89
    CROSS_ENTROPY_LOSS = 90
    CROSS_ENTROPY_LOSS_BACK = 91
    OPT_STEP_ADAMW = 92
    OPT_STEP_SGD = 93
    GLU = 94


GENERIC_OPERATION_COUNT = 95


class BinaryOp(enum.IntEnum):
    ADD = 0
    SUB = 1
    MUL = 2
    DIV = 3


class CView(ctypes.Structure):
    """emel_tensor_view / emel_tensor_view_mut (identical layouts)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("ne", ctypes.c_uint64 * 4),
        ("nb", ctypes.c_uint64 * 4),
        ("data_bytes", ctypes.c_uint64),
    ]


class CGenericRequest(ctypes.Structure):
    """emel_generic_request: the pinned generic operation struct."""

    _fields_ = [
        ("operation", ctypes.c_uint32),
        ("unary_subop", ctypes.c_uint32),
        ("glu_subop", ctypes.c_uint32),
        ("pool_subop", ctypes.c_uint32),
        ("src0", ctypes.POINTER(CView)),
        ("src1", ctypes.POINTER(CView)),
        ("src2", ctypes.POINTER(CView)),
        ("dst", ctypes.POINTER(CView)),
        ("op_params", ctypes.c_uint8 * 64),
        ("op_params_size", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("index_out", ctypes.c_void_p),
    ]


class CIndexView(ctypes.Structure):
    """emel_index_view: an int32 index tensor (IndexView, get_rows.rs:42-196)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("len", ctypes.c_uint64),
        ("ne", ctypes.c_uint64 * 3),
        ("nb", ctypes.c_uint64 * 3),
        ("explicit_strides", ctypes.c_uint32),
        ("on_host", ctypes.c_uint32),
    ]


class CSampleRequest(ctypes.Structure):
    """emel_sample_temperature_top_k_request (SampleTemperatureTopK, emel-logits sampler/sm.rs:148-195)."""

    _fields_ = [
        ("card", ctypes.c_uint64),
        ("temperature", ctypes.c_float),
        ("reserved", ctypes.c_uint32),
        ("top_k", ctypes.c_uint64),
        ("logits", ctypes.c_void_p),
        ("logits_len", ctypes.c_uint64),
        ("sorted_indices", ctypes.c_void_p),
        ("sorted_indices_len", ctypes.c_uint64),
        ("top_probabilities", ctypes.c_void_p),
        ("top_probabilities_len", ctypes.c_uint64),
        ("top_indices", ctypes.c_void_p),
        ("top_indices_len", ctypes.c_uint64),
        ("random_state", ctypes.c_void_p),
        ("selected_token_out", ctypes.c_void_p),
        ("selected_score_out", ctypes.c_void_p),
        ("status_out", ctypes.c_void_p),
    ]


class CSampleRows(ctypes.Structure):
    """emel_sample_rows: a batch of independent sampler requests."""

    _fields_ = [
        ("rows", ctypes.c_uint64),
        ("logits_stride", ctypes.c_uint64),
        ("sorted_stride", ctypes.c_uint64),
        ("top_stride", ctypes.c_uint64),
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
    "emel_op_unary_event": [ctypes.c_uint32, _V, _V, _S],
    "emel_op_log": [_V, _V, _S],
    "emel_op_sin": [_V, _V, _S],
    "emel_op_cos": [_V, _V, _S],
    "emel_op_clamp": [_V, _V, ctypes.c_float, ctypes.c_float, _S],
    "emel_op_leaky_relu": [_V, _V, ctypes.c_float, _S],
    "emel_op_silu_back": [_V, _V, _V, _S],
    "emel_op_add1": [_V, ctypes.c_float, _V, _S],
    "emel_op_acc": [_V, _V, _V, ctypes.c_uint64, _S],
    "emel_op_diag": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, _S],
    "emel_op_diag_mask_inf": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32, _S],
    "emel_op_diag_mask_zero": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32, _S],
    "emel_op_group_norm": [_V, _V, ctypes.c_uint64, ctypes.c_float, _S],
    "emel_op_l2_norm": [_V, _V, _S],
    "emel_op_argmax_rows_no_alloc": [_V, _V, _S],
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
    "emel_stream_reserve": [_S, ctypes.c_uint64, ctypes.c_uint64],
    "emel_stream_workspace": [_S, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
    "emel_device_prepare": [_S],
    "emel_stream_copy": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, _S],
    "emel_generic_dispatch": [ctypes.POINTER(CGenericRequest), _S],
    **{f"emel_op_get_rows{suffix}": [_V, ctypes.POINTER(CIndexView), _V, _S]
       for suffix in ("", "_f32_bytes", "_f16", "_bf16", "_q4_0", "_q8_0", "_q4_k")},
    "emel_sample_temperature_top_k": [ctypes.POINTER(CSampleRequest), _S],
    "emel_sample_temperature_top_k_rows": [ctypes.POINTER(CSampleRequest), ctypes.POINTER(CSampleRows), _S],
    "emel_sample_preselected": [ctypes.c_uint64, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32)],
    "emel_logits_validator_build": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32, ctypes.c_void_p,
                                    ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32,
                                    ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32), _S],
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


class CopyShape(enum.IntEnum):
    """emel_copy_shape: the streaming shapes emel_stream_copy measures."""
    FLAT = 0
    WAVE4 = 1
    WAVE8 = 2
    WALK = 3


def stream_reserve(work_bytes: int, counter_bytes: int, stream: int = 0) -> Status:
    """emel_stream_reserve: grows the scratch calls on `stream` share so later
    calls needing no more allocate nothing (refused under capture)."""
    return Status(load().emel_stream_reserve(ctypes.c_void_p(stream), work_bytes, counter_bytes))


def stream_workspace(stream: int = 0) -> tuple:
    """emel_stream_workspace: (status, work bytes, counter bytes) the stream holds now."""
    w, c = ctypes.c_uint64(0), ctypes.c_uint64(0)
    st = Status(load().emel_stream_workspace(ctypes.c_void_p(stream), ctypes.byref(w), ctypes.byref(c)))
    return st, w.value, c.value


def device_prepare(stream: int = 0) -> Status:
    """emel_device_prepare: builds the current device's tables (GELU's) and waits."""
    return Status(load().emel_device_prepare(ctypes.c_void_p(stream)))


def stream_copy(src_ptr: int, dst_ptr: int, nbytes: int, shape: "CopyShape", stream: int = 0) -> Status:
    """emel_stream_copy: a bit copy of nbytes device bytes with one streaming
    shape (a measurement reference; asynchronous on `stream`)."""
    return Status(load().emel_stream_copy(ctypes.c_void_p(src_ptr), ctypes.c_void_p(dst_ptr), nbytes, int(shape),
                                          ctypes.c_void_p(stream)))
