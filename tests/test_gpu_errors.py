"""GPU: rejected requests return the reference's error variant and leave dst
untouched (tests/any/binary_ops.rs:167, softmax_ops.rs:76-102,
normalization_ops.rs:124-160, reductions.rs:152-189 in the reference)."""
import numpy as np
import pytest
import torch

import emel_hip as eh
from helpers import Pair

pytestmark = pytest.mark.gpu

S = eh.Status
SENTINEL = np.uint32(0x7FC00001).view(np.float32)


def dev(n, fill=None, ne=None, nb=None, dtype=None, gpu=None):
    buf = np.full(n, SENTINEL if fill is None else fill, np.float32)
    return Pair(buf, ne or [n, 1, 1, 1], nb, dtype).to(gpu)


def untouched(p):
    got = p.result()
    assert (got.view(np.uint32) == p.host.view(np.uint32)).all(), "dst was written by a rejected request"


def test_binary_rejections(gpu):
    a = dev(4, 1.0, gpu=gpu)
    b = dev(4, 2.0, gpu=gpu)
    o = dev(3, ne=[3, 1, 1, 1], gpu=gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpDiv(a.pview(), b.pview(), o.pview(mut=True))) == S.SHAPE_MISMATCH
    untouched(o)
    # out of bounds: data_bytes smaller than the span
    o4 = dev(4, gpu=gpu)
    short = Pair(o4.host, [4, 1, 1, 1], None, None, data_bytes=12)
    short.dev = o4.dev
    assert k.process_event(eh.OpAdd(a.pview(), b.pview(), short.pview(mut=True))) == S.INVALID_VIEW
    untouched(o4)
    # F16 dtype on an F32 op, misaligned stride, zero stride on a non-singleton dim
    bad_dtype = Pair(a.host, [4, 1, 1, 1], dtype=eh.DType.F16)
    bad_dtype.dev = a.dev
    assert k.process_event(eh.OpAdd(bad_dtype.pview(), b.pview(), o4.pview(mut=True))) == S.INVALID_VIEW
    odd = Pair(a.host, [2, 1, 1, 1], [6, 12, 12, 12])
    odd.dev = a.dev
    o2 = dev(2, ne=[2, 1, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpAdd(odd.pview(), odd.pview(), o2.pview(mut=True))) == S.INVALID_VIEW
    zero = Pair(a.host, [2, 2, 1, 1], [4, 0, 16, 16])
    zero.dev = a.dev
    assert k.process_event(eh.OpAdd(zero.pview(), a.pview(), o4.pview(mut=True))) == S.INVALID_VIEW
    untouched(o4)
    untouched(o2)


def test_partial_overlap_is_rejected(gpu):
    buf = dev(64, 1.0, gpu=gpu)
    src = Pair(buf.host, [32, 1, 1, 1])
    src.dev = buf.dev
    dst = Pair(buf.host[8:40], [32, 1, 1, 1])
    dst.dev = buf.dev[8:40]
    before = buf.result().copy()
    assert eh.Kernel().process_event(eh.OpAdd(src.pview(), src.pview(), dst.pview(mut=True))) == S.INVALID_VIEW
    assert (buf.result() == before).all()


def test_broadcast_rejections(gpu):
    a = dev(6, 1.0, ne=[3, 2, 1, 1], gpu=gpu)
    row = dev(2, 1.0, ne=[2, 1, 1, 1], gpu=gpu)
    o = dev(6, ne=[3, 2, 1, 1], gpu=gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpAddBroadcastRow(a.pview(), row.pview(), o.pview(mut=True))) == S.SHAPE_MISMATCH
    one = dev(3, 1.0, ne=[3, 1, 1, 1], gpu=gpu)
    row3 = dev(3, 1.0, ne=[3, 1, 1, 1], gpu=gpu)
    o1 = dev(3, ne=[3, 1, 1, 1], gpu=gpu)
    # a single row is not a broadcast (dst count must exceed the row's)
    assert k.process_event(eh.OpMulBroadcastRow(one.pview(), row3.pview(), o1.pview(mut=True))) == S.SHAPE_MISMATCH
    # 4-D broadcast: src1 extent must divide dst extent
    s1 = dev(4, 1.0, ne=[1, 4, 1, 1], gpu=gpu)
    o2 = dev(6, ne=[3, 2, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpBinaryBroadcast(eh.BinaryOp.MUL, a.pview(), s1.pview(), o2.pview(mut=True))) == S.SHAPE_MISMATCH
    untouched(o)
    untouched(o1)
    untouched(o2)


def test_unary_rejections(gpu):
    a = dev(4, 1.0, gpu=gpu)
    o = dev(3, ne=[3, 1, 1, 1], gpu=gpu)
    k = eh.Kernel()
    # OpUnary reports every failed guard as UnexpectedEvent
    assert k.process_event(eh.OpUnary(eh.UnarySubOp.SILU, a.pview(), o.pview(mut=True))) == S.UNEXPECTED_EVENT
    o4 = dev(4, gpu=gpu)
    assert k.process_event(eh.OpUnary(eh.UnarySubOp.SIGMOID, a.pview(), o4.pview(mut=True))) == S.UNEXPECTED_EVENT
    assert k.process_event(eh.OpUnary(eh.UnarySubOp.HARDSWISH, a.pview(), o4.pview(mut=True))) == S.UNEXPECTED_EVENT
    # the dedicated events classify
    assert k.process_event(eh.OpSilu(a.pview(), o.pview(mut=True))) == S.SHAPE_MISMATCH
    bad = Pair(a.host, [2, 2, 1, 1], [4, 0, 16, 16])
    bad.dev = a.dev
    assert k.process_event(eh.OpGelu(bad.pview(), o4.pview(mut=True))) == S.INVALID_VIEW
    untouched(o)
    untouched(o4)


def test_norm_rejections(gpu):
    a = dev(6, 1.0, ne=[3, 2, 1, 1], gpu=gpu)
    o = dev(6, ne=[3, 2, 1, 1], gpu=gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpRmsNorm(a.pview(), o.pview(mut=True), float("nan"))) == S.INVALID_PARAMETERS
    assert k.process_event(eh.OpRmsNorm(a.pview(), o.pview(mut=True), -1.0)) == S.INVALID_PARAMETERS
    assert k.process_event(eh.OpNorm(a.pview(), o.pview(mut=True), float("inf"))) == S.INVALID_PARAMETERS
    o2 = dev(6, ne=[2, 3, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpRmsNorm(a.pview(), o2.pview(mut=True), 1.0)) == S.SHAPE_MISMATCH
    empty = Pair(a.host, [3, 0, 1, 1], [4, 12, 0, 0])
    empty.dev = a.dev
    assert k.process_event(eh.OpNorm(empty.pview(), empty.pview(mut=True), 1.0)) == S.INVALID_VIEW
    # fused weight: a one-row input fails the broadcast-row contract
    w = dev(3, 1.0, ne=[3, 1, 1, 1], gpu=gpu)
    one = dev(3, 1.0, ne=[3, 1, 1, 1], gpu=gpu)
    o1 = dev(3, ne=[3, 1, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpRmsNormMul(one.pview(), w.pview(), o1.pview(mut=True), 1.0)) == S.SHAPE_MISMATCH
    untouched(o)
    untouched(o2)
    untouched(o1)


def test_reduction_rejections(gpu):
    x = dev(6, 1.0, ne=[3, 2, 1, 1], gpu=gpu)
    k = eh.Kernel()
    o = dev(4, ne=[2, 2, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpSoftMax(x.pview(), o.pview(mut=True))) == S.SHAPE_MISMATCH
    s = dev(2, ne=[2, 1, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpSum(x.pview(), s.pview(mut=True))) == S.SHAPE_MISMATCH
    assert k.process_event(eh.OpArgmax(x.pview(), s.pview(mut=True))) == S.SHAPE_MISMATCH
    r = dev(3, ne=[1, 3, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpSumRows(x.pview(), r.pview(mut=True))) == S.SHAPE_MISMATCH
    i = Pair(np.full(2, -9, np.int32), [1, 2, 1, 1]).to(gpu)
    f = Pair(np.full(2, -9, np.int32), [1, 2, 1, 1], dtype=eh.DType.F32).to(gpu)
    assert k.process_event(eh.OpArgmaxRows(x.pview(), f.pview(mut=True))) == S.INVALID_VIEW
    bad_mask = Pair(np.zeros(6, np.uint16), [3, 2, 1, 1], dtype=eh.DType.F32).to(gpu)
    o6 = dev(6, ne=[3, 2, 1, 1], gpu=gpu)
    assert k.process_event(eh.OpSoftMaxExt(x.pview(), bad_mask.pview(), 1.0, o6.pview(mut=True))) == S.INVALID_VIEW
    m2 = Pair(np.zeros(4, np.uint16), [2, 2, 1, 1], dtype=eh.DType.F16).to(gpu)
    assert k.process_event(eh.OpSoftMaxExt(x.pview(), m2.pview(), 1.0, o6.pview(mut=True))) == S.SHAPE_MISMATCH
    for p in (o, s, r, o6):
        untouched(p)
    assert (i.result() == -9).all() and (f.result() == -9).all()
    torch.cuda.synchronize()
