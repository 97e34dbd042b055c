"""GPU parity of the generic wire envelope (emel_generic_dispatch) with the
oracle's restatement of generic.rs, through the C ABI.

Bit-exact for every route except sum and mean, whose f64 accumulation runs
as a parallel tree on the device (relative 1e-6 on the f32 result), and
norm / rms_norm rows of at least 64 columns, whose f64 row sums run as a
fixed-order tree over a workgroup (within north_star's 1e-5 relative
tolerance for rms_norm; rows narrower than 64 keep the reference's order
and are compared bit for bit).  The
documented divergences are asserted explicitly: self-overlapping
destinations are UNSUPPORTED_OPERATION, a partial last element
(the reference panics) is INVALID_SHAPE, dst overlapping a source is
INVALID_ARGUMENT."""
import struct

import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from helpers import Pair, assert_bits_equal, assert_close_rel, normal, rng, uniform

pytestmark = pytest.mark.gpu

G = eh.GenericOp
U = eh.UnarySubOp


def f32p(*v):
    return b"".join(struct.pack("=f", x) for x in v)


def i32p(*v):
    return b"".join(struct.pack("=i", x) for x in v)


def specials(n, seed):
    x = normal(seed, n) * np.float32(4)
    sp = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-40, 88.7, -104.0, 1e30, -1e30],
                  np.float32)
    x[: min(n, sp.size)] = sp[: min(n, sp.size)]
    return x


def permuted(buf, ne):
    """ne's dims 1 and 2 swapped in memory: returns nb."""
    phys = [ne[0], ne[2], ne[1], ne[3]]
    nb = [4]
    for d in range(1, 4):
        nb.append(nb[-1] * phys[d - 1])
    return [nb[0], nb[2], nb[1], nb[3]]


class Run:
    def __init__(self, gpu):
        self.gpu = gpu
        self.kernel = eh.Kernel()

    def pair(self, buf, ne, nb=None, dtype=None, data_bytes=None):
        return Pair(buf, ne, nb, dtype, data_bytes).to(self.gpu)

    def __call__(self, op, s0=None, s1=None, s2=None, d=None, params=b"", size=None, unary=0, index=False,
                 compare=True, rtol=None):
        import torch

        print(f"generic {G(op).name} unary={unary} params={params.hex()} "
              f"d={None if d is None else (d.ne, d.nb)}", flush=True)
        idx_h = np.full(1, -7, np.int32) if index else None
        want = orc.generic(op, *(p.oview() if p is not None else None for p in (s0, s1, s2, d)), params, size, unary,
                           idx_h)
        req = eh.GenericRequest(op, *(p.pview() if p is not None else None for p in (s0, s1, s2)),
                                d.pview(True) if d is not None else None,
                                eh.OpParams(params, len(params) if size is None else size)).with_unary(unary)
        idx_d = None
        if index:
            idx_d = torch.full((1,), -7, dtype=torch.int32, device=self.gpu)
            req.with_index_out(idx_d)
        got = self.kernel.process_event(eh.GenericEvent(req))
        if compare and want == orc.OK:
            assert got == eh.Status.OK, (G(op).name, got, eh.last_error())
            if rtol is None:
                assert_bits_equal(d.result(), d.host, G(op).name)
            else:
                r = d.result()
                assert (np.isnan(r) == np.isnan(d.host)).all(), G(op).name
                assert_close_rel(r, d.host, rtol, G(op).name)
            if index:
                assert int(idx_d.cpu()[0]) == int(idx_h[0])
        return want, got


@pytest.fixture(scope="module")
def run(gpu):
    return Run(gpu)


# ---- elementwise family ------------------------------------------------------------

LAYOUTS = ["dense", "permuted", "ordinal", "implicit"]


def ew_views(run, kind, seed, n2=False):
    ne = [24, 6, 5, 2]
    n = int(np.prod(ne))
    a = specials(n, seed)
    b = specials(n, seed + 1)[::-1].copy()
    if kind == "dense":
        return run.pair(a, ne), run.pair(b, ne), run.pair(np.zeros(n, np.float32), ne)
    if kind == "permuted":
        return run.pair(a, ne, permuted(a, ne)), run.pair(b, ne), run.pair(np.zeros(n, np.float32), ne)
    if kind == "ordinal":  # equal counts, different shapes
        return (run.pair(a, [48, 3, 5, 2]), run.pair(b, [8, 90, 1, 2]),
                run.pair(np.zeros(n, np.float32), ne))
    return run.pair(a, ne, [0, 0, 0, 0]), run.pair(b, ne, [0, 0, 0, 0]), run.pair(np.zeros(n, np.float32), ne,
                                                                             [0, 0, 0, 0])


# silu_back needs three equal shapes, so it has no ordinal-paired case
@pytest.mark.parametrize("op,kind", [(op, kind) for op in (G.ADD, G.SUB, G.MUL, G.DIV, G.SILU_BACK)
                                     for kind in LAYOUTS if not (op == G.SILU_BACK and kind == "ordinal")])
def test_binary_routes(run, op, kind):
    a, b, d = ew_views(run, kind, 10)
    assert run(op, a, b, None, d) == (orc.OK, eh.Status.OK)


@pytest.mark.parametrize("kind", LAYOUTS)
@pytest.mark.parametrize("op,params", [(G.DUP, b""), (G.ADD1, f32p(0.75)), (G.SCALE, f32p(-0.0883883)),
                                       (G.LEAKY_RELU, f32p(0.01)), (G.CLAMP, f32p(-1.5, 2.0)), (G.SQR, b""),
                                       (G.SQRT, b"")])
def test_unary_routes(run, op, params, kind):
    a, _, d = ew_views(run, kind, 20)
    assert run(op, a, None, None, d, params) == (orc.OK, eh.Status.OK)


@pytest.mark.parametrize("kind", LAYOUTS)
@pytest.mark.parametrize("sub", [U.ABS, U.NEG, U.TANH, U.ELU, U.RELU, U.GELU, U.SILU, U.EXP])
def test_unary_subops(run, sub, kind):
    a, _, d = ew_views(run, kind, 30)
    assert run(G.UNARY, a, None, None, d, unary=int(sub)) == (orc.OK, eh.Status.OK)


def test_dense_large_unary_and_gelu_range(run):
    n = (1 << 20) + 3
    x = np.linspace(-20, 20, n).astype(np.float32)
    for sub in (U.GELU, U.TANH, U.SILU):
        assert run(G.UNARY, run.pair(x, [n, 1, 1, 1]), None, None, run.pair(np.zeros(n, np.float32), [n, 1, 1, 1]),
                   unary=int(sub)) == (orc.OK, eh.Status.OK)


def test_repeat(run):
    src = normal(40, 3 * 2 * 4 * 1)
    for sne, dne in (([3, 2, 4, 1], [6, 4, 4, 3]), ([3, 1, 1, 1], [3, 70, 2, 1]), ([1, 2, 1, 1], [64, 4, 3, 2])):
        s = run.pair(src[: int(np.prod(sne))].copy(), sne)
        d = run.pair(np.zeros(int(np.prod(dne)), np.float32), dne)
        assert run(G.REPEAT, s, None, None, d) == (orc.OK, eh.Status.OK)


# ---- rows ------------------------------------------------------------------------


# only soft_max pairs source and dst by element count (a reshaped dst)
@pytest.mark.parametrize("op,layout", [(op, layout) for op in (G.CUMSUM, G.SOFT_MAX, G.NORM, G.RMS_NORM)
                                       for layout in ("dense", "permuted", "dst_reshaped")
                                       if layout != "dst_reshaped" or op == G.SOFT_MAX])
def test_row_routes(run, op, layout):
    ne = [37, 40, 3, 1]  # 120 rows: two workgroups of lanes
    n = int(np.prod(ne))
    x = normal(50, n) * np.float32(3)
    x[5] = np.nan
    x[37 * 7 + 3] = -np.inf
    s = run.pair(x, ne, permuted(x, ne) if layout == "permuted" else None)
    if layout == "dst_reshaped":
        d = run.pair(np.zeros(n, np.float32), [74, 20, 3, 1])
    else:
        d = run.pair(np.zeros(n, np.float32), ne)
    params = f32p(1e-5) if op in (G.NORM, G.RMS_NORM) else b""
    assert run(op, s, None, None, d, params) == (orc.OK, eh.Status.OK)


@pytest.mark.parametrize("ne,dne", [([300, 20, 1, 1], [600, 10, 1, 1]), ([5000, 3, 2, 1], [5000, 3, 2, 1])])
def test_wide_softmax_permuted_and_reshaped(run, ne, dne):
    # soft_max's exact sequential f32 sum over a workgroup per row
    n = int(np.prod(ne))
    x = normal(56, n) * np.float32(4)
    x[7] = np.nan if ne[0] == 300 else x[7]
    s = run.pair(x, ne, permuted(x, ne))
    assert run(G.SOFT_MAX, s, None, None, run.pair(np.zeros(n, np.float32), dne)) == (orc.OK, eh.Status.OK)


def test_wide_softmax_and_norm_rows(run):
    ne = [4096, 70, 1, 1]
    n = int(np.prod(ne))
    x = normal(51, n) * np.float32(5)
    for op, params in ((G.SOFT_MAX, b""), (G.RMS_NORM, f32p(1e-6)), (G.NORM, f32p(0.0))):
        assert run(op, run.pair(x, ne), None, None, run.pair(np.zeros(n, np.float32), ne), params,
                   rtol=None if op == G.SOFT_MAX else 1e-5) == (orc.OK, eh.Status.OK)


@pytest.mark.parametrize("op", [G.RMS_NORM, G.NORM])
@pytest.mark.parametrize("ne,layout", [([4096, 2048, 1, 1], "dense"),      # config 3's shape: 256-thread rows
                                       ([1000, 30, 4, 1], "permuted"),     # 64-thread rows, permuted rows
                                       ([64, 33, 2, 1], "dense"),          # the narrowest workgroup rows
                                       ([63, 33, 2, 1], "dense"),          # one lane per row, bit for bit
                                       ([3000, 12, 1, 1], "strided")])     # dim 0 strided by 3 floats
def test_norm_rows_workgroup(run, op, ne, layout):
    n = int(np.prod(ne))
    if layout == "strided":
        x = normal(57, 3 * n) * np.float32(3)
        nb = [12, 12 * ne[0], 12 * ne[0] * ne[1], 12 * n]
    else:
        x = normal(57, n) * np.float32(3)
        nb = permuted(x, ne) if layout == "permuted" else None
    if ne[0] == 4096:  # config 3: 1% of rows x100
        rows = np.random.Generator(np.random.PCG64(6)).choice(ne[1], 20, replace=False)
        x.reshape(ne[1], ne[0])[rows] *= np.float32(100.0)
    s = run.pair(x, ne, nb)
    d = run.pair(np.zeros(n, np.float32), ne)
    assert run(op, s, None, None, d, f32p(1e-5), rtol=None if ne[0] < 64 else 1e-5) == (orc.OK, eh.Status.OK)


@pytest.mark.parametrize("op", [G.RMS_NORM, G.NORM])
def test_norm_rows_workgroup_non_finite(run, op):
    ne = [2048, 6, 1, 1]
    x = normal(58, int(np.prod(ne))).reshape(ne[1], ne[0])
    x[0, 5] = np.nan
    x[1, 2047] = np.inf
    x[2, 0] = -np.inf
    x[2, 9] = np.inf
    x[3, :] = 0.0
    x[4, :] = np.float32(3e38)
    assert run(op, run.pair(x.reshape(-1), ne), None, None, run.pair(np.zeros(x.size, np.float32), ne), f32p(0.0),
               rtol=1e-5) == (orc.OK, eh.Status.OK)


@pytest.mark.parametrize("row", [6, 15, 60])
def test_softmax_back(run, row):
    ne = [6, 10, 3, 2]
    n = int(np.prod(ne))
    v = uniform(52, n, 0, 1)
    g = normal(53, n)
    assert run(G.SOFT_MAX_BACK, run.pair(v, ne, permuted(v, ne)), run.pair(g, ne), None,
               run.pair(np.zeros(n, np.float32), ne), i32p(row)) == (orc.OK, eh.Status.OK)


def test_rms_norm_back(run):
    ne = [33, 50, 2, 1]
    n = int(np.prod(ne))
    x, dy = normal(54, n), normal(55, n)
    assert run(G.RMS_NORM_BACK, run.pair(x, ne), run.pair(dy, ne, permuted(dy, ne)), None,
               run.pair(np.zeros(n, np.float32), ne), f32p(1e-5)) == (orc.OK, eh.Status.OK)


# ---- per-element generators and index ops --------------------------------------------


def test_fill_and_arange(run):
    n = (1 << 25) + 5  # ordinals above 2^24 round in the f32 conversion
    d = run.pair(np.zeros(n, np.float32), [n, 1, 1, 1])
    assert run(G.ARANGE, None, None, None, d, f32p(-1000.5, 0.0625)) == (orc.OK, eh.Status.OK)
    d = run.pair(np.zeros(4096, np.float32), [16, 16, 4, 4], [4, 64, 1024, 4096 * 1])
    assert run(G.FILL, None, None, None, d, f32p(-0.0)) == (orc.OK, eh.Status.OK)


def test_diag_and_masks(run):
    n = 300
    s = run.pair(normal(60, n), [n, 1, 1, 1])
    assert run(G.DIAG, s, None, None, run.pair(np.full(n * n, 5, np.float32), [n, n, 1, 1])) == (orc.OK, eh.Status.OK)
    x = normal(61, n * n)
    for op in (G.DIAG_MASK_INF, G.DIAG_MASK_ZERO):
        for n_past in (0, 17, 2**31 - 1):
            src = run.pair(x, [n, n, 1, 1], [4 * n, 4, 4 * n * n, 4 * n * n])  # transposed
            assert run(op, src, None, None, run.pair(np.zeros(n * n, np.float32), [n, n, 1, 1]), i32p(n_past)) == \
                (orc.OK, eh.Status.OK)


@pytest.mark.parametrize("axis", [0, 1, 2, 3])
def test_concat(run, axis):
    lne = [9, 4, 3, 2]
    rne = list(lne)
    rne[axis] = 5
    dne = list(lne)
    dne[axis] += 5
    lhs = normal(62, int(np.prod(lne)))
    rhs = normal(63, int(np.prod(rne)))
    assert run(G.CONCAT, run.pair(lhs, lne, permuted(lhs, lne)), run.pair(rhs, rne), None,
               run.pair(np.zeros(int(np.prod(dne)), np.float32), dne), i32p(axis)) == (orc.OK, eh.Status.OK)


def test_repeat_back(run):
    for tne, q in (([5, 3, 2, 1], [3, 2, 4, 2]), ([64, 1, 1, 1], [1, 40, 3, 1]), ([1, 1, 1, 1], [50, 3, 2, 2])):
        sne = [t * m for t, m in zip(tne, q)]
        src = normal(64, int(np.prod(sne)))
        assert run(G.REPEAT_BACK, run.pair(src, sne, permuted(src, sne)), None, None,
                   run.pair(np.zeros(int(np.prod(tne)), np.float32), tne)) == (orc.OK, eh.Status.OK)


# ---- whole-tensor reductions -----------------------------------------------------------


def test_l2_norm(run):
    for ne in ([3, 1, 1, 1], [1000, 7, 3, 1]):
        n = int(np.prod(ne))
        x = normal(70, n)
        assert run(G.L2_NORM, run.pair(x, ne, permuted(x, ne)), None, None,
                   run.pair(np.zeros(n, np.float32), ne)) == (orc.OK, eh.Status.OK)


def test_count_equal(run):
    n = 1 << 20
    a = normal(71, n)
    b = a.copy()
    b[rng(72).random(n) < 0.4] = 0.5
    b[:10] = np.nan
    a[:5] = b[:5]  # identical NaN bits count as equal
    one = lambda: run.pair(np.zeros(1, np.float32), [1, 1, 1, 1])
    assert run(G.COUNT_EQUAL, run.pair(a, [1024, 1024, 1, 1]), run.pair(b, [n, 1, 1, 1]), None, one()) == \
        (orc.OK, eh.Status.OK)
    big = (1 << 24) + 11
    z = np.zeros(big, np.float32)
    assert run(G.COUNT_EQUAL, run.pair(z, [big, 1, 1, 1]), run.pair(z, [big, 1, 1, 1]), None, one()) == \
        (orc.OK, eh.Status.OK)


def test_sum_mean_argmax(run):
    ne = [1000, 37, 3, 1]
    n = int(np.prod(ne))
    x = normal(73, n)
    x[777] = 9.0
    x[5000] = 9.0
    for op in (G.SUM, G.MEAN, G.ARGMAX):
        d = run.pair(np.zeros(1, np.float32), [1, 1, 1, 1])
        want, got = run(op, run.pair(x, ne, permuted(x, ne)), None, None, d, compare=False)
        assert want == orc.OK and got == eh.Status.OK
        if op == G.ARGMAX:
            assert_bits_equal(d.result(), d.host, "argmax")
        else:
            assert_close_rel(d.result(), d.host, 1e-6, G(op).name)


# ---- mul_mat ------------------------------------------------------------------------------


def test_mul_mat_f32(run):
    k, m, n = 300, 33, 65
    lhs = normal(80, k * m)
    rhs = normal(81, n * k)
    lnb = [4 * m, 4, 4 * k * m, 4 * k * m]  # lhs stored transposed
    assert run(G.MUL_MAT, run.pair(lhs, [k, m, 1, 1], lnb), run.pair(rhs, [n, k, 1, 1]), None,
               run.pair(np.zeros(n * m, np.float32), [n, m, 1, 1])) == (orc.OK, eh.Status.OK)


def test_mul_mat_f16(run):
    k, m, n = 128, 20, 31
    lhs = rng(82).standard_normal(k * m).astype(np.float16).view(np.uint16)
    rhs = rng(83).standard_normal(k * n).astype(np.float16).view(np.uint16)
    d = run.pair(np.zeros(2 * m * n, np.float32), [m, n, 1, 1], [4, 8 * m, 8 * m * n, 8 * m * n])  # every other column
    assert run(G.MUL_MAT, run.pair(lhs, [k, m, 1, 1]), run.pair(rhs, [k, n, 1, 1]), None, d) == (orc.OK, eh.Status.OK)


def test_mul_mat_argmax(run):
    k, rows = 256, 5000
    w = normal(84, k * rows)
    h = normal(85, k)
    w[1234 * k:1235 * k] += np.float32(0.5) * np.sign(h)  # the largest dot ...
    w[4000 * k:4001 * k] = w[1234 * k:1235 * k]  # ... tied exactly by a later row: the lower row wins
    one = lambda: run.pair(np.zeros(1, np.float32), [1, 1, 1, 1])
    assert run(G.MUL_MAT_ARGMAX, run.pair(w, [k, rows, 1, 1]), run.pair(h, [k, 1, 1, 1]), None, one(),
               index=True) == (orc.OK, eh.Status.OK)
    w0 = w.copy()
    w0[3] = np.nan
    assert run(G.MUL_MAT_ARGMAX, run.pair(w0, [k, rows, 1, 1]), run.pair(h, [k, 1, 1, 1]), None, one(),
               index=True) == (orc.OK, eh.Status.OK)


# ---- classification, divergences and aliasing ------------------------------------------


def test_rejections_match_the_oracle_and_leave_dst(run):
    a = run.pair(normal(90, 16), [4, 4, 1, 1])
    d = run.pair(np.full(16, 3.0, np.float32), [4, 4, 1, 1])
    d3 = run.pair(np.full(3, 3.0, np.float32), [3, 1, 1, 1])
    cases = [
        (G.ADD, a, a, None, d3, b""),                   # counts differ -> InvalidShape
        (G.GET_ROWS, a, None, None, d, b""),             # no maintained route -> Unsupported
        (G.RMS_NORM, a, None, None, d, f32p(-1.0)),      # negative epsilon -> InvalidShape
        (G.CONCAT, a, a, None, d, i32p(0)),              # shapes do not concatenate -> InvalidShape
    ]
    for op, s0, s1, s2, dd, p in cases:
        want, got = run(op, s0, s1, s2, dd, p)
        assert int(got) == want, (G(op).name, want, got)
    want, got = run(G.UNARY, a, None, None, d, unary=int(U.SIGMOID))
    assert want == orc.INVALID_SHAPE and got == eh.Status.INVALID_SHAPE
    assert (d3.result() == 3.0).all()


def test_log_sin_cos_routes(run):
    # f32::ln / sin / cos through the glibc replicas: bit-exact, strided too
    g = np.random.Generator(np.random.PCG64(94))
    vals = np.concatenate([g.uniform(-1e4, 1e4, 700), g.standard_normal(200) * 3, [0.0, -0.0, 1.0, -1.0, np.inf,
                           -np.inf, np.nan, 1e-40, 3e38, 120.0, -120.0, 1e9]]).astype(np.float32)
    n = vals.size
    for op in (G.LOG, G.SIN, G.COS):
        x = run.pair(vals, [n, 1, 1, 1])
        d = run.pair(np.full(n, 3.0, np.float32), [n, 1, 1, 1])
        want, got = run(op, x, None, None, d)
        assert want == orc.OK and got == eh.Status.OK, (G(op).name, want, got)
        xs = run.pair(np.repeat(vals, 2), [n // 4, 4, 1, 1], [8, 8 * (n // 4), 8 * n, 8 * n])
        ds = run.pair(np.full(n, 3.0, np.float32), [4, n // 4, 1, 1])
        want, got = run(op, xs, None, None, ds)
        assert want == orc.OK and got == eh.Status.OK, (G(op).name, want, got)


def test_divergences(run):
    x = run.pair(uniform(91, 16, 0.5, 2.0), [16, 1, 1, 1])
    d = run.pair(np.full(16, 3.0, np.float32), [16, 1, 1, 1])
    short = run.pair(uniform(92, 16), [16, 1, 1, 1], data_bytes=62)  # last element 2 bytes short
    want, got = run(G.DUP, short, None, None, d)
    assert want == orc.PANIC and got == eh.Status.INVALID_SHAPE
    overlapping = run.pair(np.full(16, 3.0, np.float32), [4, 4, 1, 1], [4, 8, 64, 64])  # rows overlap
    want, got = run(G.DUP, x, None, None, overlapping, compare=False)
    assert want == orc.OK and got == eh.Status.UNSUPPORTED_OPERATION
    assert (d.result() == 3.0).all() and (overlapping.result() == 3.0).all()


def test_in_place_and_partial_overlap(run, gpu):
    import torch

    ne = [64, 8, 1, 1]
    x = normal(93, 512)
    want = np.zeros(512, np.float32)
    assert orc.generic(G.SOFT_MAX, orc.view(x, ne), None, None, orc.view(want, ne)) == orc.OK
    t = torch.from_numpy(x.copy()).to(gpu)
    lay = eh.Layout(0, ne, [4, 256, 2048, 2048])
    req = eh.GenericRequest(G.SOFT_MAX, eh.TensorView(t, lay), None, None, eh.TensorViewMut(t, lay))
    assert run.kernel.process_event(eh.GenericEvent(req)) == eh.Status.OK
    assert_bits_equal(t.cpu().numpy(), want, "in-place soft_max")
    # dst shifted by one row over its own source: refused
    t2 = torch.from_numpy(x.copy()).to(gpu)
    half = eh.Layout(0, [64, 4, 1, 1], [4, 256, 1024, 1024])
    req = eh.GenericRequest(G.SOFT_MAX, eh.TensorView(t2, half), None, None,
                            eh.TensorViewMut(t2[64:], half, data_bytes=4 * 448))
    assert run.kernel.process_event(eh.GenericEvent(req)) == eh.Status.INVALID_ARGUMENT
    assert_bits_equal(t2.cpu().numpy(), x, "untouched")
