"""Row gather events, mirroring emel-kernels' get_rows module.

    idx = IndexView(ids, [n_tokens, 1, 1])              # IndexView::new
    status = Kernel().process_event(OpGetRows(TensorView(table, lay), idx,
                                              TensorViewMut(out, out_lay)))

IndexView(data, ne) is IndexView::new (row-major) and
IndexView.with_strides(data, ne, nb) is IndexView::with_strides
(get_rows.rs:54-85).  Sources are TensorViews whose Layout dtype selects the
format the event expects: F32 (OpGetRows, OpGetRowsF32Bytes), F16, BF16 and
the packed Q4_0 / Q8_0 / Q4_K rows (`Layout.packed`).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from .abi import CIndexView
from .views import TensorView, TensorViewMut


class IndexView:
    """An int32 index tensor with three extents (get_rows.rs:42-196).

    data is a numpy int32 array or a CPU tensor (host memory: checked in
    place and passed to the kernel by value), a GPU tensor (device memory:
    copied back once for the check), or a raw pointer with `length` and
    `on_host`."""

    def __init__(self, data, ne, nb=None, length: int | None = None, on_host: bool | None = None):
        self._keep = data
        if isinstance(data, int):
            if length is None or on_host is None:
                raise ValueError("a raw pointer needs its length in int32 elements and its location")
            self.ptr = data
            self.len = int(length)
            self.on_host = bool(on_host)
        elif hasattr(data, "__array_interface__"):  # numpy
            if data.dtype.name != "int32" or not data.flags["C_CONTIGUOUS"]:
                raise ValueError("host indices are a C-contiguous int32 array")
            self.ptr = int(data.__array_interface__["data"][0])
            self.len = data.size if length is None else int(length)
            self.on_host = True
        else:  # torch tensor
            self.ptr = int(data.data_ptr())
            avail = int(data.untyped_storage().nbytes()) // 4 - int(data.storage_offset())
            self.len = avail if length is None else int(length)
            self.on_host = not data.is_cuda
        self.ne = [int(x) for x in ne]
        self.nb = None if nb is None else [int(x) for x in nb]
        if len(self.ne) != 3 or (self.nb is not None and len(self.nb) != 3):
            raise ValueError("an index view has three extents and three byte strides")

    @classmethod
    def with_strides(cls, data, ne, nb, length: int | None = None) -> "IndexView":
        return cls(data, ne, nb, length)

    def c(self) -> CIndexView:
        v = CIndexView()
        v.data = self.ptr
        v.len = self.len
        for d in range(3):
            v.ne[d] = self.ne[d]
            v.nb[d] = 0 if self.nb is None else self.nb[d]
        v.explicit_strides = 0 if self.nb is None else 1
        v.on_host = 1 if self.on_host else 0
        return v


def _gather(fn_name):
    def _call(self, lib, s):
        return getattr(lib, fn_name)(ctypes.byref(self.source.c()), ctypes.byref(self.indices.c()),
                                     ctypes.byref(self.destination.c()), s)
    return _call


@dataclass
class OpGetRows:
    """get_rows::OpGetRows::new(src, indices, dst) (get_rows.rs:219-226, :501-509)."""

    source: TensorView
    indices: IndexView
    destination: TensorViewMut
    _call = _gather("emel_op_get_rows")


@dataclass
class OpGetRowsF32Bytes:
    """OpGetRowsF32Bytes::new (get_rows.rs:228-260): byte-addressed F32 rows."""

    source: TensorView
    indices: IndexView
    destination: TensorViewMut
    _call = _gather("emel_op_get_rows_f32_bytes")


@dataclass
class OpGetRowsF16:
    """OpGetRowsF16::new (get_rows.rs:262-273, :410-426)."""

    source: TensorView
    indices: IndexView
    destination: TensorViewMut
    _call = _gather("emel_op_get_rows_f16")


@dataclass
class OpGetRowsBf16:
    """OpGetRowsBf16::new (get_rows.rs:386-408)."""

    source: TensorView
    indices: IndexView
    destination: TensorViewMut
    _call = _gather("emel_op_get_rows_bf16")


@dataclass
class OpGetRowsQ4_0:
    """OpGetRowsQ4_0::new (get_rows.rs:427-451)."""

    source: TensorView
    indices: IndexView
    destination: TensorViewMut
    _call = _gather("emel_op_get_rows_q4_0")


@dataclass
class OpGetRowsQ8_0:
    """OpGetRowsQ8_0::new (get_rows.rs:452-476)."""

    source: TensorView
    indices: IndexView
    destination: TensorViewMut
    _call = _gather("emel_op_get_rows_q8_0")


@dataclass
class OpGetRowsQ4K:
    """OpGetRowsQ4K::new (get_rows.rs:477-499)."""

    source: TensorView
    indices: IndexView
    destination: TensorViewMut
    _call = _gather("emel_op_get_rows_q4_k")
