"""The generic wire envelope, mirroring emel-kernels' event::GenericEvent.

    request = (GenericRequest(GenericOp.SOFT_MAX, TensorView(x, lay), None, None,
                              TensorViewMut(y, lay), OpParams.empty()))
    status = Kernel().process_event(GenericEvent(request))

GenericRequest carries the arguments of GenericRequest::new (generic.rs:
660-681) and its builders with_unary / with_glu / with_pool /
with_index_out (:683-710); GenericEvent hands it to emel_generic_dispatch,
which runs the reference machine's generic transitions (sm.rs:318-426).
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass, field

from .abi import CGenericRequest, GenericOp, GluSubOp, UnarySubOp


class OpParams:
    """OpParams (generic.rs:575-625): 64 bytes and an initialised prefix length."""

    SIZE = 64

    def __init__(self, data: bytes = b"", length: int | None = None):
        data = bytes(data)
        if len(data) > self.SIZE:
            raise ValueError("op_params holds at most 64 bytes")
        self.bytes = data.ljust(self.SIZE, b"\0")
        self.len = len(data) if length is None else int(length)
        if not 0 <= self.len <= self.SIZE:
            raise ValueError("OpParams::new rejects lengths beyond 64")

    @classmethod
    def empty(cls) -> "OpParams":
        return cls(b"", 0)

    @classmethod
    def f32(cls, *values: float) -> "OpParams":
        """Consecutive native-endian f32 slots (parameter_f32, generic.rs:935-939)."""
        return cls(b"".join(struct.pack("=f", float(v)) for v in values))

    @classmethod
    def i32(cls, *values: int) -> "OpParams":
        """Consecutive native-endian i32 slots (parameter_i32, generic.rs:941-945)."""
        return cls(b"".join(struct.pack("=i", int(v)) for v in values))

    def as_slice(self) -> bytes:
        return self.bytes[: self.len]


@dataclass
class GenericRequest:
    """GenericRequest::new(operation, src0, src1, src2, dst, params); the
    selectors default as the reference's do (pool Avg, unary Abs, glu ReGlu)."""

    operation: int
    src0: object = None
    src1: object = None
    src2: object = None
    dst: object = None
    params: OpParams = field(default_factory=OpParams.empty)
    unary: int = int(UnarySubOp.ABS)
    glu: int = int(GluSubOp.REGLU)
    pool: int = 1  # PoolSubOp::Avg (pool.rs:18-23)
    index_out: object = None  # device int32 tensor (one element) or raw device pointer

    def with_unary(self, subop: int) -> "GenericRequest":
        self.unary = int(subop)
        return self

    def with_glu(self, subop: int) -> "GenericRequest":
        self.glu = int(subop)
        return self

    def with_pool(self, subop: int) -> "GenericRequest":
        self.pool = int(subop)
        return self

    def with_index_out(self, index_out) -> "GenericRequest":
        self.index_out = index_out
        return self

    def c(self) -> CGenericRequest:
        r = CGenericRequest()
        r.operation = int(self.operation)
        r.unary_subop = self.unary
        r.glu_subop = self.glu
        r.pool_subop = self.pool
        self._views = []
        for name in ("src0", "src1", "src2", "dst"):
            v = getattr(self, name)
            if v is not None:
                cv = v.c()
                self._views.append(cv)
                setattr(r, name, ctypes.pointer(cv))
        ctypes.memmove(r.op_params, self.params.bytes, OpParams.SIZE)
        r.op_params_size = self.params.len
        r.reserved = 0
        if self.index_out is None:
            r.index_out = None
        elif isinstance(self.index_out, int):
            r.index_out = self.index_out
        else:
            r.index_out = int(self.index_out.data_ptr())
        return r


@dataclass
class GenericEvent:
    """event::GenericEvent::new(request) (generic.rs:797-830)."""

    request: GenericRequest

    def operation(self) -> GenericOp:
        return GenericOp(self.request.operation)

    def _call(self, lib, s):
        req = self.request.c()
        return lib.emel_generic_dispatch(ctypes.byref(req), s)
