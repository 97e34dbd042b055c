"""GPU: emel_op_argmax_rows_no_alloc, the allocation-free variant of
emel_op_argmax_rows, called through the C ABI.  Its indices must equal the
existing entry point's bit for bit (and the oracle's) on consecutive calls
that reuse the device's static scratch: a large request, then smaller ones,
then shapes that take the two-level merge and the single-workgroup path."""
import ctypes

import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from helpers import Pair

pytestmark = pytest.mark.gpu


def logits(cols, rows, seed):
    """N(0,1) rows, a planted maximum per row, a tie at a higher index in
    even rows, and a NaN in column 0 of row 1 (its result is 0)."""
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal(cols * rows, dtype=np.float64).astype(np.float32).reshape(rows, cols)
    where = g.integers(0, cols, rows)
    for r in range(rows):
        x[r, where[r]] = np.float32(9.0 + r * 1e-3)
        if r % 2 == 0 and where[r] + 1 < cols:
            x[r, g.integers(where[r] + 1, cols)] = x[r, where[r]]
    if rows > 1 and cols > 1:
        x[1, 0] = np.nan
    return x.reshape(-1)


def call(lib, name, a, ne, gpu):
    rows = int(np.prod(ne[1:]))
    o = Pair(np.full(rows, -7, np.int32), [1, ne[1], ne[2], ne[3]]).to(gpu)
    status = getattr(lib, name)(ctypes.byref(a.pview().c()), ctypes.byref(o.pview(mut=True).c()), None)
    assert status == eh.Status.OK, (name, eh.last_error())
    assert lib.emel_stream_synchronize(None) == eh.Status.OK
    return o.result()


def check(lib, gpu, cols, rows, seed):
    ne = [cols, rows, 1, 1]
    print(f"no_alloc argmax_rows cols={cols} rows={rows} seed={seed}", flush=True)
    a = Pair(logits(cols, rows, seed), ne).to(gpu)
    got = call(lib, "emel_op_argmax_rows_no_alloc", a, ne, gpu)
    ref = call(lib, "emel_op_argmax_rows", a, ne, gpu)
    assert (got == ref).all(), (np.flatnonzero(got != ref)[:5], got[got != ref][:5], ref[got != ref][:5])
    want = np.full(rows, -7, np.int32)
    assert orc.argmax_rows(a.oview(), orc.view(want, [1, rows, 1, 1])) == orc.OK
    assert (got == want).all()
    return got


def test_no_alloc_matches_argmax_rows_on_consecutive_calls(gpu):
    lib = eh.load()
    check(lib, gpu, 151936, 64, 701)   # config 5: 32 chunks per row
    check(lib, gpu, 4095, 3, 702)      # smaller, scalar rows, 4 chunks per row
    check(lib, gpu, 1 << 21, 1, 703)   # one long row: groups of 64 chunks, two-level merge
    check(lib, gpu, 1000, 2500, 704)   # rows >= 2048: one workgroup per row, no scratch
    check(lib, gpu, 151936, 64, 705)   # config 5 again after the others


def test_no_alloc_rejects_like_argmax_rows(gpu):
    lib = eh.load()
    a = Pair(logits(64, 4, 706), [64, 4, 1, 1]).to(gpu)
    bad = Pair(np.full(5, -7, np.int32), [1, 5, 1, 1]).to(gpu)  # dst rows != src rows
    for name in ("emel_op_argmax_rows_no_alloc", "emel_op_argmax_rows"):
        status = getattr(lib, name)(ctypes.byref(a.pview().c()), ctypes.byref(bad.pview(mut=True).c()), None)
        assert status == eh.Status.SHAPE_MISMATCH, name
    assert (bad.result() == -7).all()
