"""Layout and tensor views mirroring emel-kernels' tensor_view.rs.

`Layout(dtype, ne, nb)` is the pinned wire shape (tensor_view.rs:215-219):
four extents and four byte strides, nb[0] == 0 meaning implicit row-major.
`TensorView` / `TensorViewMut` bind a layout to device memory.  The memory
comes from a torch tensor (plumbing only): the view's data pointer is the
tensor's first element and data_bytes is the rest of the tensor's storage
from there, which is what the Rust slice length expresses for the
reference's bounds check.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

from .abi import CView, DType

_ELEM = {DType.F32: 4, DType.F16: 2, DType.I32: 4, DType.BF16: 2}
# Packed formats: (values per block, bytes per block) (quant.rs:13-17, quant_more.rs:38-48).
_PACKED = {DType.Q4_0: (32, 18), DType.Q8_0: (32, 34), DType.Q4_K: (256, 144)}


@dataclass(frozen=True)
class Layout:
    dtype: int
    ne: tuple
    nb: tuple

    def __init__(self, dtype: int, ne: Sequence[int], nb: Sequence[int]):
        object.__setattr__(self, "dtype", int(dtype))
        object.__setattr__(self, "ne", tuple(int(x) for x in ne))
        object.__setattr__(self, "nb", tuple(int(x) for x in nb))
        if len(self.ne) != 4 or len(self.nb) != 4:
            raise ValueError("a layout has exactly four extents and four byte strides")

    @staticmethod
    def contiguous(dtype: int, ne: Sequence[int]) -> "Layout":
        """Layout::contiguous (tensor_view.rs:229-240): row-major strides of
        4-byte elements whatever the dtype, as the reference builds them."""
        nb = [4]
        for d in range(1, 4):
            nb.append(nb[-1] * int(ne[d - 1]))
        return Layout(dtype, ne, nb)

    @staticmethod
    def dense(dtype: int, ne: Sequence[int]) -> "Layout":
        """Row-major strides of the dtype's own element size (f16 masks)."""
        nb = [_ELEM.get(int(dtype), 4)]
        for d in range(1, 4):
            nb.append(nb[-1] * int(ne[d - 1]))
        return Layout(dtype, ne, nb)

    @staticmethod
    def packed(dtype: int, ne: Sequence[int]) -> "Layout":
        """Packed quantized rows: nb = [1, row bytes, ...] as PackedRowView
        requires (tensor_view.rs:487-532)."""
        values, block_bytes = _PACKED[DType(int(dtype))]
        row = (int(ne[0]) // values) * block_bytes
        nb = [1, row, row * int(ne[1]), row * int(ne[1]) * int(ne[2])]
        return Layout(dtype, ne, nb)

    def permuted(self, axes: Sequence[int]) -> "Layout":
        """Layout::permuted (tensor_view.rs:285-300): dim d takes source axes[d]."""
        return Layout(self.dtype, [self.ne[a] for a in axes], [self.nb[a] for a in axes])

    def element_count(self) -> int:
        c = 1
        for e in self.ne:
            c *= e
        return c


def _storage_bytes_from(tensor) -> int:
    """Bytes of the tensor's storage from its first element to the end."""
    storage = tensor.untyped_storage()
    return int(storage.nbytes()) - int(tensor.storage_offset()) * tensor.element_size()


class _View:
    def __init__(self, data, layout: Layout, data_bytes: int | None = None):
        self.layout = layout
        self._keep = data
        if isinstance(data, int):
            if data_bytes is None:
                raise ValueError("a raw device pointer needs data_bytes")
            self.ptr = data
            self.data_bytes = int(data_bytes)
        else:
            self.ptr = int(data.data_ptr())
            self.data_bytes = _storage_bytes_from(data) if data_bytes is None else int(data_bytes)

    def c(self) -> CView:
        v = CView()
        v.data = self.ptr
        v.data_bytes = self.data_bytes
        v.dtype = self.layout.dtype
        v.reserved = 0
        for d in range(4):
            v.ne[d] = self.layout.ne[d]
            v.nb[d] = self.layout.nb[d]
        return v


class TensorView(_View):
    """Immutable view (TensorView::new(data, layout), tensor_view.rs:690-701)."""


class TensorViewMut(_View):
    """Mutable view (TensorViewMut::new(data, layout), tensor_view.rs:812-823)."""
