"""CPU: emel_generic_dispatch classifies requests on the host exactly as the
oracle's restatement of the reference machine does (sm.rs:318-426), over
randomly mutated requests for every maintained operation.  Without a GPU an
accepted request stops at the device check (KERNEL_UNAVAILABLE), so no
kernel runs and the host buffers are only read by the oracle."""
import ctypes
import struct

import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from emel_hip.abi import CGenericRequest, CView

OK, INVALID_ARGUMENT, INVALID_SHAPE, UNSUPPORTED = 0, 8, 9, 10
KERNEL_UNAVAILABLE = int(eh.Status.KERNEL_UNAVAILABLE)
G = eh.GenericOp
TWO_SOURCE = {G.ADD, G.SUB, G.MUL, G.DIV, G.SILU_BACK, G.CONCAT, G.SOFT_MAX_BACK, G.RMS_NORM_BACK, G.COUNT_EQUAL,
              G.MUL_MAT, G.MUL_MAT_ARGMAX}


def _no_gpu():
    return eh.device_count() == 0


pytestmark = pytest.mark.skipif(not _no_gpu(), reason="host-pointer requests only run where no GPU is visible")


class Spec:
    """A view description: ne, nb, dtype, data_bytes (None = exact span)."""

    def __init__(self, ne, nb=None, dtype=0, data_bytes=None):
        self.ne = list(ne)
        elem = 2 if dtype == 1 else 4
        if nb is None:
            nb = [elem]
            for d in range(1, 4):
                nb.append(nb[-1] * self.ne[d - 1])
        self.nb = list(nb)
        self.dtype = dtype
        self.data_bytes = data_bytes

    def strides(self):
        if self.dtype == 0 and self.nb[0] == 0:
            st = [4]
            for d in range(1, 4):
                st.append(st[-1] * self.ne[d - 1])
            return st
        return self.nb

    def span(self):
        st = self.strides()
        return sum((max(n, 1) - 1) * s for n, s in zip(self.ne, st)) + (2 if self.dtype == 1 else 4)


def base_request(op, g):
    """A request the op's maintained route accepts."""
    a = [int(x) for x in g.integers(1, 4, 4)]
    p = b""
    s0 = s1 = None
    d = Spec(a)
    unary = 0
    idx = True
    f = lambda *v: b"".join(struct.pack("=f", x) for x in v)
    i = lambda *v: b"".join(struct.pack("=i", x) for x in v)
    if op in (G.ADD, G.SUB, G.MUL, G.DIV):
        s0, s1 = Spec(a), Spec(a[::-1])
    elif op in (G.DUP, G.SQR, G.SQRT, G.LOG, G.SIN, G.COS, G.SOFT_MAX):
        s0 = Spec(a[::-1])
    elif op in (G.ADD1, G.SCALE, G.LEAKY_RELU):
        s0, p = Spec(a), f(float(g.standard_normal()))
    elif op == G.CLAMP:
        s0, p = Spec(a), f(-1.0, 1.0)
    elif op == G.SILU_BACK:
        s0, s1 = Spec(a), Spec(a)
    elif op in (G.CUMSUM, G.L2_NORM):
        s0 = Spec(a)
    elif op == G.REPEAT:
        s0 = Spec(a)
        d = Spec([x * int(g.integers(1, 3)) for x in a])
    elif op == G.REPEAT_BACK:
        s0 = Spec([x * int(g.integers(1, 3)) for x in a])
    elif op == G.CONCAT:
        ax = int(g.integers(0, 4))
        b = list(a)
        b[ax] = int(g.integers(1, 3))
        dd = list(a)
        dd[ax] += b[ax]
        s0, s1, d, p = Spec(a), Spec(b), Spec(dd), i(ax)
    elif op == G.DIAG:
        n = a[0]
        s0, d = Spec([n, 1, 1, 1]), Spec([n, n, 1, 1])
    elif op in (G.DIAG_MASK_INF, G.DIAG_MASK_ZERO):
        n = a[0]
        s0, d, p = Spec([n, n, 1, 1]), Spec([n, n, 1, 1]), i(int(g.integers(0, 3)))
    elif op == G.SOFT_MAX_BACK:
        s0, s1, p = Spec(a), Spec(a), i(a[0])
    elif op == G.RMS_NORM_BACK:
        s0, s1, p = Spec(a), Spec(a), f(1e-5)
    elif op in (G.NORM, G.RMS_NORM):
        s0, p = Spec(a), f(1e-5)
    elif op == G.COUNT_EQUAL:
        s0, s1, d = Spec(a), Spec(a[::-1]), Spec([1, 1, 1, 1])
    elif op in (G.SUM, G.MEAN, G.ARGMAX):
        s0, d = Spec(a), Spec([1, 1, 1, 1])
    elif op == G.FILL:
        p = f(2.5)
    elif op == G.ARANGE:
        p = f(1.0, 0.5)
    elif op == G.MUL_MAT:
        k, m, n = a[0], a[1], a[2]
        if g.random() < 0.5:
            s0, s1, d = Spec([k, m, 1, 1]), Spec([n, k, 1, 1]), Spec([n, m, 1, 1])
        else:
            s0, s1, d = Spec([k, m, 1, 1], dtype=1), Spec([k, n, 1, 1], dtype=1), Spec([m, n, 1, 1])
    elif op == G.MUL_MAT_ARGMAX:
        k, m = a[0], a[1]
        s0, s1, d = Spec([k, m, 1, 1]), Spec([k, 1, 1, 1]), Spec([1, 1, 1, 1])
    elif op == G.UNARY:
        s0 = Spec(a)
        unary = int(g.choice([0, 2, 4, 5, 6, 8, 10, 13]))
    else:  # no maintained route
        s0 = Spec(a)
    return dict(op=int(op), s0=s0, s1=s1, s2=None, d=d, params=p, size=len(p), unary=unary, index=idx)


def mutate(req, g):
    views = [k for k in ("s0", "s1", "s2", "d") if req[k] is not None]
    kind = int(g.integers(0, 12))
    if kind == 0 and views:  # change an extent
        v = req[str(g.choice(views))]
        v.ne[int(g.integers(0, 4))] = int(g.integers(0, 4))
        v.nb = Spec(v.ne, dtype=v.dtype).nb
    elif kind == 1 and views:  # odd strides
        v = req[str(g.choice(views))]
        v.nb[int(g.integers(0, 4))] = int(g.choice([0, 2, 4, 6, 8, 12, 16, 64]))
    elif kind == 2 and views:  # implicit row-major
        v = req[str(g.choice(views))]
        v.nb = [0, 0, 0, 0]
    elif kind == 3 and views:  # short or partial buffers
        v = req[str(g.choice(views))]
        v.data_bytes = max(0, v.span() - int(g.integers(1, 6)))
    elif kind == 4:  # drop or add a view
        k = str(g.choice(["s0", "s1", "s2", "d"]))
        req[k] = None if req[k] is not None else Spec([2, 1, 1, 1])
    elif kind == 5:  # parameter bytes
        req["size"] = int(g.integers(0, 9))
    elif kind == 6:
        req["params"] = b"".join(struct.pack("=f", float(x)) for x in g.choice(
            [np.nan, np.inf, -1.0, 0.0, 2.0, -3.0], 2))
        req["size"] = 8
    elif kind == 7:
        req["params"] = b"".join(struct.pack("=i", int(x)) for x in g.integers(-2, 5, 2))
        req["size"] = 8
    elif kind == 8:
        req["unary"] = int(g.integers(0, 22))
    elif kind == 9 and views:  # dtype
        v = req[str(g.choice(views))]
        v.dtype = int(g.choice([0, 1, 26, 30]))
    elif kind == 10:
        req["index"] = not req["index"]
    elif kind == 11 and views:  # permute two dims of a view
        v = req[str(g.choice(views))]
        i, j = g.choice(4, 2, replace=False)
        v.ne[i], v.ne[j] = v.ne[j], v.ne[i]
        v.nb[i], v.nb[j] = v.nb[j], v.nb[i]


def elements_disjoint(spec):
    st = spec.strides()
    dims = sorted([d for d in range(4) if spec.ne[d] > 1], key=lambda d: st[d])
    span = 4
    for d in dims:
        if st[d] < span:
            return False
        span += (spec.ne[d] - 1) * st[d]
    return True


def aligned(spec):
    e = 2 if spec.dtype == 1 else 4
    return all(spec.ne[d] <= 1 or spec.strides()[d] % e == 0 for d in range(4))


def expected_product(want, req):
    """The product's status given the oracle's, per the documented divergences."""
    if want not in (OK, orc.PANIC):
        return want
    op = req["op"]
    used = [req["d"]]
    if op not in (G.FILL, G.ARANGE):
        used.append(req["s0"])
    if op in TWO_SOURCE:
        used.append(req["s1"])
    if not all(aligned(v) for v in used):
        return UNSUPPORTED
    if want == orc.PANIC:
        return INVALID_SHAPE
    if not elements_disjoint(req["d"]):
        return UNSUPPORTED
    return KERNEL_UNAVAILABLE


def run(req):
    bufs = {}
    oviews = {}
    cviews = {}
    for k in ("s0", "s1", "s2", "d"):
        s = req[k]
        if s is None:
            continue
        nbytes = s.span() if s.data_bytes is None else s.data_bytes
        buf = np.zeros(max(nbytes, 1) // 4 + 16, np.float32)
        bufs[k] = buf
        oviews[k] = orc.view(buf, s.ne, s.nb, s.dtype, nbytes)
        cv = CView()
        cv.data = buf.ctypes.data
        cv.data_bytes = nbytes
        cv.dtype = s.dtype
        cv.reserved = 0
        for d in range(4):
            cv.ne[d] = s.ne[d]
            cv.nb[d] = s.nb[d]
        cviews[k] = cv
    index = np.zeros(1, np.int32)
    want = orc.generic(req["op"], oviews.get("s0"), oviews.get("s1"), oviews.get("s2"), oviews.get("d"),
                       req["params"], req["size"], req["unary"], index if req["index"] else None)
    r = CGenericRequest()
    r.operation = req["op"]
    r.unary_subop = req["unary"]
    r.glu_subop = 0
    r.pool_subop = 1
    for k, name in (("s0", "src0"), ("s1", "src1"), ("s2", "src2"), ("d", "dst")):
        if k in cviews:
            setattr(r, name, ctypes.pointer(cviews[k]))
    ctypes.memmove(r.op_params, bytes(req["params"]).ljust(64, b"\0"), 64)
    r.op_params_size = req["size"]
    r.index_out = index.ctypes.data if req["index"] else None
    got = eh.load().emel_generic_dispatch(ctypes.byref(r), None)
    return want, got


MAINTAINED = [G.DUP, G.ADD, G.SUB, G.MUL, G.DIV, G.ADD1, G.SCALE, G.LEAKY_RELU, G.CLAMP, G.SILU_BACK, G.CUMSUM,
              G.REPEAT, G.REPEAT_BACK, G.CONCAT, G.DIAG, G.DIAG_MASK_INF, G.DIAG_MASK_ZERO, G.SOFT_MAX_BACK,
              G.RMS_NORM_BACK, G.L2_NORM, G.COUNT_EQUAL, G.FILL, G.ARANGE, G.MUL_MAT, G.MUL_MAT_ARGMAX, G.SQR, G.SQRT,
              G.LOG, G.SIN, G.COS, G.SUM, G.MEAN, G.ARGMAX, G.SOFT_MAX, G.NORM, G.RMS_NORM, G.UNARY]


@pytest.mark.parametrize("op", MAINTAINED + [G.GET_ROWS, G.ROPE, G.GLU, G.SUM_ROWS])
def test_dispatch_classification_matches_the_oracle(op):
    g = np.random.Generator(np.random.PCG64(1000 + int(op)))
    seen = set()
    for trial in range(300):
        req = base_request(op, g)
        for _ in range(int(g.integers(0, 3)) if trial else 0):
            mutate(req, g)
        want, got = run(req)
        exp = expected_product(want, req)
        assert got == exp, (G(op).name, trial, want, got, {k: (vars(v) if v else None) for k, v in req.items()
                                                          if k in ("s0", "s1", "d")}, req["params"], req["size"])
        seen.add(want)
    if op in MAINTAINED:
        assert OK in seen and INVALID_SHAPE in seen, seen
    else:
        assert UNSUPPORTED in seen, seen


def test_unrepresentable_requests_are_invalid_arguments():
    lib = eh.load()
    assert lib.emel_generic_dispatch(None, None) == INVALID_ARGUMENT
    base = base_request(G.ADD, np.random.Generator(np.random.PCG64(1)))
    for field, value in (("operation", 95), ("unary_subop", 22), ("glu_subop", 6), ("pool_subop", 2),
                         ("op_params_size", 65), ("reserved", 1)):
        r = CGenericRequest()
        r.operation = G.ADD
        r.pool_subop = 1
        setattr(r, field, value)
        assert lib.emel_generic_dispatch(ctypes.byref(r), None) == INVALID_ARGUMENT, field
    assert base["op"] == G.ADD


def test_struct_layout():
    assert ctypes.sizeof(CGenericRequest) == 128
    assert CGenericRequest.op_params.offset == 48
    assert CGenericRequest.index_out.offset == 120


# ---- row gather: host-side classification against the oracle ---------------------------


def test_get_rows_classification_matches_the_oracle():
    """Views, shapes and strides are classified on the host before the index
    check, which needs the device: an oracle OK or INDEX_OUT_OF_BOUNDS is
    KERNEL_UNAVAILABLE here."""
    from emel_hip.abi import CIndexView

    g = np.random.Generator(np.random.PCG64(77))
    lib = eh.load()
    kinds = [(orc.GR_F32, 0, "emel_op_get_rows", 4), (orc.GR_F32_BYTES, 0, "emel_op_get_rows_f32_bytes", 4),
             (orc.GR_F16, 1, "emel_op_get_rows_f16", 2), (orc.GR_BF16, 30, "emel_op_get_rows_bf16", 2),
             (orc.GR_Q4_0, 2, "emel_op_get_rows_q4_0", 0), (orc.GR_Q8_0, 8, "emel_op_get_rows_q8_0", 0),
             (orc.GR_Q4_K, 12, "emel_op_get_rows_q4_k", 0)]
    seen = {}
    for trial in range(3000):
        kind, dtype, fn, elem = kinds[trial % len(kinds)]
        cols = {2: 32, 8: 32, 12: 256}.get(dtype, int(g.integers(1, 5)))
        rows = int(g.integers(1, 4))
        ine = [int(g.integers(0, 3)), int(g.integers(1, 3)), int(g.integers(1, 3))]
        sne = [cols, rows, ine[1], ine[2]]
        if dtype in (2, 8, 12):
            bv, bb = {2: (32, 18), 8: (32, 34), 12: (256, 144)}[dtype]
            row = cols // bv * bb
            snb = [1, row, row * rows, row * rows * ine[1]]
        else:
            snb = [elem]
            for d in range(1, 4):
                snb.append(snb[-1] * sne[d - 1])
        dne = [cols, ine[0], ine[1], ine[2]]
        dnb = [4, 4 * dne[0], 4 * dne[0] * dne[1], 4 * dne[0] * dne[1] * dne[2]]
        inb = None
        idx_len = int(np.prod(ine))
        # mutations
        m = int(g.integers(0, 10))
        if m == 0:
            sne[int(g.integers(0, 4))] = int(g.integers(0, 4))
        elif m == 1:
            snb[int(g.integers(0, 4))] = int(g.choice([0, 1, 2, 3, 4, 6, 8, 9]))
        elif m == 2:
            snb[0] = 0
        elif m == 3:
            dne[int(g.integers(0, 4))] = int(g.integers(0, 4))
        elif m == 4:
            dnb[int(g.integers(0, 4))] = int(g.choice([0, 4, 8]))
        elif m == 5:
            inb = [int(g.choice([0, 2, 4, 8, 12])) for _ in range(3)]
        elif m == 6:
            idx_len = max(0, idx_len - int(g.integers(1, 3)))
        elif m == 7:
            ine[int(g.integers(0, 3))] = int(g.integers(0, 4))
        src_span = 1
        for d in range(4):
            src_span += max(sne[d] - 1, 0) * snb[d]
        src_bytes = max(src_span + 8, cols * 4 + 8) if m != 8 else max(src_span - 2, 0)
        src = np.zeros(max(src_bytes, 8) // 4 + 4, np.float32)
        count = int(np.prod(dne))
        out = np.zeros(max(count, 1) + 4, np.float32)
        idx = np.zeros(max(idx_len, 1), np.int32)
        want = orc.get_rows(kind, orc.view(src, sne, snb, dtype, src_bytes),
                            orc.index_view(idx[:idx_len] if idx_len else np.zeros(0, np.int32), ine, inb, idx_len),
                            orc.view(out, dne, dnb, 0, 4 * count))
        cs, cd = CView(), CView()
        for v, arr, ne, nb, dt, nbytes in ((cs, src, sne, snb, dtype, src_bytes), (cd, out, dne, dnb, 0, 4 * count)):
            v.data = arr.ctypes.data
            v.data_bytes = nbytes
            v.dtype = dt
            v.reserved = 0
            for d in range(4):
                v.ne[d] = ne[d]
                v.nb[d] = nb[d]
        ci = CIndexView()
        ci.data = idx.ctypes.data
        ci.len = idx_len
        for d in range(3):
            ci.ne[d] = ine[d]
            ci.nb[d] = 0 if inb is None else inb[d]
        ci.explicit_strides = 0 if inb is None else 1
        ci.on_host = int(trial % 2)  # host-resident and device-resident indices classify alike before the check
        got = getattr(lib, fn)(ctypes.byref(cs), ctypes.byref(ci), ctypes.byref(cd), None)
        expect = KERNEL_UNAVAILABLE if want in (OK, orc.INDEX_OUT_OF_BOUNDS) else want
        assert got == expect, (trial, kind, want, got, sne, snb, ine, inb, idx_len, dne, dnb, src_bytes)
        seen[want] = seen.get(want, 0) + 1
    assert {OK, orc.INVALID_VIEW, orc.SHAPE_MISMATCH} <= set(seen), seen
