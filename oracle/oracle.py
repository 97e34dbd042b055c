"""ctypes binding of the CPU oracle (oracle/libemel_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker the HIP product is compared against.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.

Views are host numpy arrays with the reference's (ne, nb) wire layout;
`data_bytes` defaults to the array's byte length (the Rust slice length).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libemel_oracle.so"

OK, INVALID_VIEW, SHAPE_MISMATCH, INVALID_PARAMETERS, UNEXPECTED_EVENT = 0, 1, 2, 3, 4
INVALID_SHAPE = 9
INVALID_OFFSET, ZERO_NORM = 15, 16
ADD, SUB, MUL, DIV = 0, 1, 2, 3
F32, F16, I32 = 0, 1, 26


class OView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("ne", ctypes.c_uint64 * 4),
        ("nb", ctypes.c_uint64 * 4),
        ("data_bytes", ctypes.c_uint64),
    ]


def view(arr: np.ndarray, ne, nb=None, dtype: int | None = None, data_bytes: int | None = None) -> OView:
    """A host view over a C-contiguous numpy array.  nb=None -> row-major of
    the array's element size; keep `arr` alive while the view is used."""
    if not arr.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle views need C-contiguous backing arrays")
    if dtype is None:
        dtype = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.uint16): F16,
                 np.dtype(np.int32): I32}[arr.dtype]
    ne = [int(x) for x in ne]
    if nb is None:
        nb = [arr.itemsize]
        for d in range(1, 4):
            nb.append(nb[-1] * ne[d - 1])
    v = OView()
    v.data = arr.ctypes.data
    v.data_bytes = arr.nbytes if data_bytes is None else int(data_bytes)
    v.dtype = dtype
    v.reserved = 0
    for d in range(4):
        v.ne[d] = ne[d]
        v.nb[d] = int(nb[d])
    v._arr = arr  # keep alive
    return v


_P = ctypes.POINTER(OView)
_SIG = {
    "orc_layout_validate": [_P, ctypes.c_int],
    "orc_normalization_view_valid": [_P],
    "orc_op_binary": [ctypes.c_int, _P, _P, _P],
    "orc_op_broadcast_row": [ctypes.c_int, _P, _P, _P],
    "orc_op_unary": [ctypes.c_int, _P, _P],
    "orc_op_unary_event": [ctypes.c_int, _P, _P],
    "orc_op_log": [_P, _P],
    "orc_op_sin": [_P, _P],
    "orc_op_cos": [_P, _P],
    "orc_op_clamp": [_P, _P, ctypes.c_float, ctypes.c_float],
    "orc_op_leaky_relu": [_P, _P, ctypes.c_float],
    "orc_op_silu_back": [_P, _P, _P],
    "orc_op_add1": [_P, ctypes.c_float, _P],
    "orc_op_acc": [_P, _P, _P, ctypes.c_uint64],
    "orc_op_diag": [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64],
    "orc_op_diag_mask": [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32],
    "orc_op_group_norm": [_P, _P, ctypes.c_uint64, ctypes.c_float],
    "orc_op_l2_norm": [_P, _P],
    "orc_op_scale": [_P, _P, ctypes.c_float],
    "orc_op_rms_norm": [_P, _P, ctypes.c_float],
    "orc_op_norm": [_P, _P, ctypes.c_float],
    "orc_op_soft_max": [_P, _P],
    "orc_op_sum_rows": [_P, _P],
    "orc_op_sum": [_P, _P],
    "orc_op_mean": [_P, _P],
    "orc_op_argmax": [_P, _P],
    "orc_op_repeat": [_P, _P],
    "orc_soft_max_ext": [_P, _P, ctypes.c_float, _P],
    "orc_argmax_rows": [_P, _P],
    "orc_binary_bcast": [ctypes.c_int, _P, _P, _P],
    "orc_rms_norm_mul": [_P, _P, _P, ctypes.c_float],
    "orc_swiglu": [_P, _P, _P],
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIG.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        for name in ("orc_silu", "orc_gelu"):
            getattr(L, name).argtypes = [ctypes.c_float]
            getattr(L, name).restype = ctypes.c_float
        for name in ("orc_slice_dup",):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64]
            getattr(L, name).restype = ctypes.c_int
        L.orc_slice_power.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64]
        L.orc_slice_power.restype = ctypes.c_int
        L.orc_slice_binary.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64,
                                       ctypes.c_void_p, ctypes.c_uint64]
        L.orc_slice_binary.restype = ctypes.c_int
        L.orc_op_glu.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64]
        L.orc_op_glu.restype = ctypes.c_int
        L.orc_glu_gate.argtypes = [ctypes.c_int, ctypes.c_float]
        L.orc_glu_gate.restype = ctypes.c_float
        L.orc_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.orc_fp32_to_fp16.restype = ctypes.c_uint16
        L.orc_fp16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_fp16_to_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _r(v):
    return None if v is None else ctypes.byref(v)


def call(name: str, *args) -> int:
    """Calls orc_<name> with OView arguments passed by reference."""
    fn = getattr(lib(), name)
    conv = [_r(a) if isinstance(a, OView) or a is None else a for a in args]
    return int(fn(*conv))


# convenience wrappers -------------------------------------------------------

def binary(op, lhs, rhs, dst): return call("orc_op_binary", op, lhs, rhs, dst)
def broadcast_row(op, src0, src1, dst): return call("orc_op_broadcast_row", op, src0, src1, dst)
def unary(subop, src, dst): return call("orc_op_unary", subop, src, dst)
def unary_event(subop, src, dst): return call("orc_op_unary_event", subop, src, dst)
def log(src, dst): return call("orc_op_log", src, dst)
def sin(src, dst): return call("orc_op_sin", src, dst)
def cos(src, dst): return call("orc_op_cos", src, dst)
def clamp(src, dst, lo, hi): return call("orc_op_clamp", src, dst, ctypes.c_float(lo), ctypes.c_float(hi))
def leaky_relu(src, dst, slope): return call("orc_op_leaky_relu", src, dst, ctypes.c_float(slope))
def silu_back(src, grad, dst): return call("orc_op_silu_back", src, grad, dst)
def add1(src, scalar, dst): return call("orc_op_add1", src, ctypes.c_float(scalar), dst)
def acc(base, update, dst, offset): return call("orc_op_acc", base, update, dst, ctypes.c_uint64(offset))
def group_norm(src, dst, groups, eps): return call("orc_op_group_norm", src, dst, ctypes.c_uint64(groups), ctypes.c_float(eps))
def l2_norm(src, dst): return call("orc_op_l2_norm", src, dst)


def diag(inp: np.ndarray, out: np.ndarray) -> int:
    return int(lib().orc_op_diag(inp.ctypes.data, inp.size, out.ctypes.data, out.size))


def diag_mask(inf: bool, inp: np.ndarray, out: np.ndarray, n_past: int) -> int:
    return int(lib().orc_op_diag_mask(int(inf), inp.ctypes.data, inp.size, out.ctypes.data, out.size, n_past))
def scale(src, dst, s): return call("orc_op_scale", src, dst, ctypes.c_float(s))
def rms_norm(src, dst, eps): return call("orc_op_rms_norm", src, dst, ctypes.c_float(eps))
def norm(src, dst, eps): return call("orc_op_norm", src, dst, ctypes.c_float(eps))
def soft_max(src, dst): return call("orc_op_soft_max", src, dst)
def sum_rows(src, dst): return call("orc_op_sum_rows", src, dst)
def sum_(src, dst): return call("orc_op_sum", src, dst)
def mean(src, dst): return call("orc_op_mean", src, dst)
def argmax(src, dst): return call("orc_op_argmax", src, dst)
def repeat(src, dst): return call("orc_op_repeat", src, dst)
def soft_max_ext(src, mask, s, dst): return call("orc_soft_max_ext", src, mask, ctypes.c_float(s), dst)
def argmax_rows(src, dst): return call("orc_argmax_rows", src, dst)
def binary_bcast(op, src0, src1, dst): return call("orc_binary_bcast", op, src0, src1, dst)
def rms_norm_mul(src, w, dst, eps): return call("orc_rms_norm_mul", src, w, dst, ctypes.c_float(eps))
def swiglu(gate, up, dst): return call("orc_swiglu", gate, up, dst)
def _f32p(a):
    assert a.dtype == np.float32
    return a.ctypes.data


def slice_dup(inp, out, in_len=None, out_len=None) -> int:
    return int(lib().orc_slice_dup(_f32p(inp), inp.size if in_len is None else in_len, _f32p(out),
                                   out.size if out_len is None else out_len))


def slice_binary(op, lhs, rhs, out) -> int:
    return int(lib().orc_slice_binary(op, _f32p(lhs), lhs.size, _f32p(rhs), rhs.size, _f32p(out), out.size))


def slice_power(sqrt_, inp, out) -> int:
    return int(lib().orc_slice_power(1 if sqrt_ else 0, _f32p(inp), inp.size, _f32p(out), out.size))


def op_power(sqrt_, src, dst): return call("orc_op_power", 1 if sqrt_ else 0, src, dst)


REGLU, GEGLU, SWIGLU, SWIGLU_OAI, GEGLU_ERF, GEGLU_QUICK = 0, 1, 2, 3, 4, 5


def glu(subop, inp: np.ndarray, out: np.ndarray, input_len=None, output_len=None) -> int:
    """OpGlu over host float32 arrays (lengths default to the arrays')."""
    assert inp.dtype == np.float32 and out.dtype == np.float32
    return int(lib().orc_op_glu(subop, inp.ctypes.data, inp.size if input_len is None else input_len,
                                out.ctypes.data, out.size if output_len is None else output_len))


def glu_gate(subop, g: float) -> float: return float(lib().orc_glu_gate(subop, g))
def silu_scalar(x: float) -> float: return float(lib().orc_silu(x))
def gelu_scalar(x: float) -> float: return float(lib().orc_gelu(x))
def fp32_to_fp16(x: float) -> int: return int(lib().orc_fp32_to_fp16(x))
def fp16_to_f32(h: int) -> float: return float(lib().orc_fp16_to_f32(h))


# generic wire envelope --------------------------------------------------------

UNSUPPORTED_OPERATION, INVALID_ARGUMENT, PANIC = 10, 8, 99


class OGenericRequest(ctypes.Structure):
    """orc_generic_request (the emel_generic_request layout, host pointers)."""

    _fields_ = [
        ("operation", ctypes.c_uint32),
        ("unary_subop", ctypes.c_uint32),
        ("glu_subop", ctypes.c_uint32),
        ("pool_subop", ctypes.c_uint32),
        ("src0", ctypes.POINTER(OView)),
        ("src1", ctypes.POINTER(OView)),
        ("src2", ctypes.POINTER(OView)),
        ("dst", ctypes.POINTER(OView)),
        ("op_params", ctypes.c_uint8 * 64),
        ("op_params_size", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("index_out", ctypes.c_void_p),
    ]


def generic(operation: int, src0=None, src1=None, src2=None, dst=None, params: bytes = b"",
            params_size: int | None = None, unary: int = 0, index_out: np.ndarray | None = None) -> int:
    """orc_generic over OView arguments; params are the op_params bytes
    (params_size defaults to their length); index_out is a 1-element int32
    host array or None."""
    r = OGenericRequest()
    r.operation = int(operation)
    r.unary_subop = int(unary)
    r.glu_subop = 0
    r.pool_subop = 1
    for name, v in (("src0", src0), ("src1", src1), ("src2", src2), ("dst", dst)):
        if v is not None:
            setattr(r, name, ctypes.pointer(v))
    raw = bytes(params).ljust(64, b"\0")
    ctypes.memmove(r.op_params, raw, 64)
    r.op_params_size = len(params) if params_size is None else int(params_size)
    r.reserved = 0
    if index_out is not None:
        assert index_out.dtype == np.int32 and index_out.size >= 1
        r.index_out = index_out.ctypes.data
    L = lib()
    L.orc_generic.argtypes = [ctypes.POINTER(OGenericRequest)]
    L.orc_generic.restype = ctypes.c_int
    return int(L.orc_generic(ctypes.byref(r)))


# row gather -------------------------------------------------------------------

INDEX_OUT_OF_BOUNDS, UNSUPPORTED_SOURCE_STRIDE = 11, 12
GR_F32, GR_F32_BYTES, GR_F16, GR_BF16, GR_Q4_0, GR_Q8_0, GR_Q4_K = range(7)


class OIndexView(ctypes.Structure):
    """orc_index_view (the emel_index_view layout, host pointer)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("len", ctypes.c_uint64),
        ("ne", ctypes.c_uint64 * 3),
        ("nb", ctypes.c_uint64 * 3),
        ("explicit_strides", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


def index_view(arr: np.ndarray, ne, nb=None, length: int | None = None) -> OIndexView:
    """IndexView::new(arr, ne) when nb is None, else IndexView::with_strides."""
    assert arr.dtype == np.int32 and arr.flags["C_CONTIGUOUS"]
    v = OIndexView()
    v.data = arr.ctypes.data if arr.size else 0
    v.len = arr.size if length is None else int(length)
    for d in range(3):
        v.ne[d] = int(ne[d])
        v.nb[d] = 0 if nb is None else int(nb[d])
    v.explicit_strides = 0 if nb is None else 1
    v.reserved = 0
    v._arr = arr
    return v


def get_rows(kind: int, src: OView, idx: OIndexView, dst: OView) -> int:
    L = lib()
    L.orc_get_rows.argtypes = [ctypes.c_int, ctypes.POINTER(OView), ctypes.POINTER(OIndexView), ctypes.POINTER(OView)]
    L.orc_get_rows.restype = ctypes.c_int
    return int(L.orc_get_rows(kind, ctypes.byref(src), ctypes.byref(idx), ctypes.byref(dst)))


# ---- emel-logits sampler and validator (emel_oracle_sampler.c) ----------------

INVALID_REQUEST = 13


def _sampler_lib():
    L = lib()
    if not getattr(L, "_sampler_sigs", False):
        L.orc_park_miller_next.argtypes = [ctypes.c_uint32]
        L.orc_park_miller_next.restype = ctypes.c_uint32
        L.orc_sampler_softmax.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_uint64]
        L.orc_sampler_softmax.restype = ctypes.c_float
        L.orc_sample_temperature_top_k.argtypes = [
            ctypes.c_uint64, ctypes.c_float, ctypes.c_uint64,
            ctypes.POINTER(ctypes.c_float), ctypes.c_uint64, ctypes.POINTER(ctypes.c_int32), ctypes.c_uint64,
            ctypes.POINTER(ctypes.c_float), ctypes.c_uint64, ctypes.POINTER(ctypes.c_int32), ctypes.c_uint64,
            ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_float)]
        L.orc_sample_temperature_top_k.restype = ctypes.c_int
        L.orc_validator_build.argtypes = [
            ctypes.POINTER(ctypes.c_float), ctypes.c_uint64, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32),
            ctypes.c_uint64, ctypes.POINTER(ctypes.c_float), ctypes.c_uint64, ctypes.c_int32,
            ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]
        L.orc_validator_build.restype = ctypes.c_int
        L._sampler_sigs = True
    return L


def _ptr(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def park_miller_next(state: int) -> int:
    return int(_sampler_lib().orc_park_miller_next(state))


def sampler_softmax(values: np.ndarray) -> float:
    """In place over a float32 array; returns the sequential f32 sum."""
    return float(_sampler_lib().orc_sampler_softmax(_ptr(values, ctypes.c_float), values.size))


def sample_temperature_top_k(card, temperature, top_k, logits, sorted_indices, top_probabilities, top_indices,
                             random_state, selected, score, lens=None):
    """Sampler::sample_temperature_top_k over numpy buffers (modified in place).
    random_state / selected / score are 1-element uint32 / int32 / float32
    arrays.  lens overrides the (logits, sorted, top_p, top_i) lengths."""
    if lens is None:
        lens = (logits.size, sorted_indices.size, top_probabilities.size, top_indices.size)
    return int(_sampler_lib().orc_sample_temperature_top_k(
        card, ctypes.c_float(temperature), top_k, _ptr(logits, ctypes.c_float), lens[0],
        _ptr(sorted_indices, ctypes.c_int32), lens[1], _ptr(top_probabilities, ctypes.c_float), lens[2],
        _ptr(top_indices, ctypes.c_int32), lens[3], _ptr(random_state, ctypes.c_uint32),
        _ptr(selected, ctypes.c_int32), _ptr(score, ctypes.c_float)))


def validator_build(logits, vocab_size, ids, scores, capacity, count_out, error_out, lens=None):
    """Validator::process_event(Build) over numpy buffers; count_out and
    error_out are 1-element int32 arrays (error: 0 None, 1 InvalidRequest)."""
    if lens is None:
        lens = (logits.size, ids.size, scores.size)
    return int(_sampler_lib().orc_validator_build(
        _ptr(logits, ctypes.c_float), lens[0], vocab_size, _ptr(ids, ctypes.c_int32), lens[1],
        _ptr(scores, ctypes.c_float), lens[2], capacity, _ptr(count_out, ctypes.c_int32),
        _ptr(error_out, ctypes.c_int32)))
