"""CPU: pins the oracle with checks independent of its own code: numpy's IEEE
float32 arithmetic and strided views (np.lib.stride_tricks), numpy's f16
conversion, float64 closed forms, and the special cases the compositions
must reduce to.  A dropped term, wrong index or swapped operand in the
oracle fails one of these."""
import math

import numpy as np
import pytest
from numpy.lib.stride_tricks import as_strided

import oracle as orc
from helpers import bits, normal, uniform

OPS = {orc.ADD: np.add, orc.SUB: np.subtract, orc.MUL: np.multiply, orc.DIV: np.divide}


def np_view(buf, ne, nb):
    """The logical tensor of a (ne, nb) view as a numpy array in ordinal order."""
    if nb[0] == 0:
        nb = [4, 4 * ne[0], 4 * ne[0] * ne[1], 4 * ne[0] * ne[1] * ne[2]]
    return as_strided(buf, shape=tuple(reversed(ne)), strides=tuple(reversed(nb))).reshape(-1)


def random_strided(g, ne):
    """A backing buffer and explicit byte strides (padded, possibly permuted)."""
    order = g.permutation(4)
    nb = [0] * 4
    step = 4 * int(g.integers(1, 3))
    for d in order:
        nb[d] = step
        step *= ne[d] + int(g.integers(0, 2))
    span = sum((ne[d] - 1) * nb[d] for d in range(4)) // 4 + 1
    return g.standard_normal(span).astype(np.float32), nb


@pytest.mark.parametrize("seed", range(40))
def test_binary_matches_numpy_on_strided_views(seed):
    g = np.random.Generator(np.random.PCG64(seed))
    ne = [int(x) for x in g.integers(1, 6, 4)]
    op = int(g.integers(0, 4))
    a, anb = random_strided(g, ne)
    b, bnb = random_strided(g, ne)
    # the output may have a different shape with the same count
    one = ne[0] * ne[1]
    one_ne = [one, ne[2], ne[3], 1]
    o, onb = random_strided(g, one_ne)
    o = o.copy()
    assert orc.binary(op, orc.view(a, ne, anb), orc.view(b, ne, bnb), orc.view(o, one_ne, onb)) == orc.OK
    with np.errstate(all="ignore"):
        want = OPS[op](np_view(a, ne, anb), np_view(b, ne, bnb)).astype(np.float32)
    got = np_view(o, one_ne, onb)
    assert (bits(got) == bits(want)).all()


def test_binary_special_values_match_numpy():
    vals = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, 3.4e38, -3.4e38, 0.1, 7.0], np.float32)
    a = np.repeat(vals, vals.size)
    b = np.tile(vals, vals.size)
    n = a.size
    for op, fn in OPS.items():
        out = np.zeros(n, np.float32)
        assert orc.binary(op, orc.view(a, [n, 1, 1, 1]), orc.view(b, [n, 1, 1, 1]), orc.view(out, [n, 1, 1, 1])) == orc.OK
        with np.errstate(all="ignore"):
            want = fn(a, b)
        same = (bits(out) == bits(want)) | (np.isnan(out) & np.isnan(want))
        assert same.all(), op


@pytest.mark.parametrize("ne0,rows", [(3, 2), (17, 5), (64, 3)])
def test_broadcast_row_matches_numpy(ne0, rows):
    a = uniform(1, ne0 * rows)
    r = uniform(2, ne0)
    for op in (orc.ADD, orc.MUL):
        out = np.zeros_like(a)
        assert orc.broadcast_row(op, orc.view(a, [ne0, rows, 1, 1]), orc.view(r, [ne0, 1, 1, 1]),
                                 orc.view(out, [ne0, rows, 1, 1])) == orc.OK
        want = OPS[op](a.reshape(rows, ne0), r[None, :]).reshape(-1)
        assert (bits(out) == bits(want)).all()


@pytest.mark.parametrize("seed", range(20))
def test_repeat_matches_numpy_tile(seed):
    g = np.random.Generator(np.random.PCG64(100 + seed))
    src_ne = [int(x) for x in g.integers(1, 4, 4)]
    reps = [int(x) for x in g.integers(1, 4, 4)]
    dst_ne = [s * r for s, r in zip(src_ne, reps)]
    src = g.standard_normal(int(np.prod(src_ne))).astype(np.float32)
    dst = np.zeros(int(np.prod(dst_ne)), np.float32)
    assert orc.repeat(orc.view(src, src_ne), orc.view(dst, dst_ne)) == orc.OK
    want = np.tile(src.reshape(tuple(reversed(src_ne))), tuple(reversed(reps))).reshape(-1)
    assert (bits(dst) == bits(want)).all()


def test_binary_bcast_special_cases():
    ne0, rows = 48, 6
    a = uniform(3, ne0 * rows)
    r = uniform(4, ne0)
    out1 = np.zeros_like(a)
    out2 = np.zeros_like(a)
    # src1 = [ne0,1,1,1] reduces to OpMulBroadcastRow
    assert orc.binary_bcast(orc.MUL, orc.view(a, [ne0, rows, 1, 1]), orc.view(r, [ne0, 1, 1, 1]),
                            orc.view(out1, [ne0, rows, 1, 1])) == orc.OK
    assert orc.broadcast_row(orc.MUL, orc.view(a, [ne0, rows, 1, 1]), orc.view(r, [ne0, 1, 1, 1]),
                             orc.view(out2, [ne0, rows, 1, 1])) == orc.OK
    assert (bits(out1) == bits(out2)).all()
    # equal shapes reduce to OpMul
    b = uniform(5, ne0 * rows)
    assert orc.binary_bcast(orc.SUB, orc.view(a, [ne0, rows, 1, 1]), orc.view(b, [ne0, rows, 1, 1]),
                            orc.view(out1, [ne0, rows, 1, 1])) == orc.OK
    assert (bits(out1) == bits(a - b)).all()
    # permuted src0 (config 5b's shape class) against numpy broadcasting
    sne = [8, 4, 6, 2]
    storage = normal(6, int(np.prod(sne)))
    nb = [4, 32, 128, 768]
    vne = [8, 6, 4, 2]
    vnb = [nb[0], nb[2], nb[1], nb[3]]
    s1 = uniform(7, 8 * 4, 0.5, 1.5)  # [8, 1, 4, 1]
    out = np.zeros(int(np.prod(vne)), np.float32)
    assert orc.binary_bcast(orc.MUL, orc.view(storage, vne, vnb), orc.view(s1, [8, 1, 4, 1]),
                            orc.view(out, vne)) == orc.OK
    x = np_view(storage, vne, vnb).reshape(2, 4, 6, 8)
    want = (x * s1.reshape(1, 4, 1, 8)).reshape(-1)
    assert (bits(out) == bits(want)).all()


def test_fp16_conversion_matches_numpy():
    g = np.random.Generator(np.random.PCG64(9))
    xs = np.concatenate([g.standard_normal(20000).astype(np.float32) * 100,
                         np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 6.1035156e-05, 5.96e-8, 2.98e-8,
                                   2.9802322e-08, np.inf, -np.inf], np.float32),
                         g.standard_normal(5000).astype(np.float32) * 1e-6])
    for x in xs:
        with np.errstate(over="ignore"):
            want = np.float32(x).astype(np.float16).view(np.uint16)
        assert orc.fp32_to_fp16(float(x)) == want, x
    for h in range(0, 65536, 7):
        f16 = np.uint16(h).view(np.float16)
        got = orc.fp16_to_f32(h)
        if np.isnan(f16):
            assert math.isnan(got)
        else:
            assert np.float32(got) == np.float32(f16)


def test_gelu_outputs_are_fp16_values_and_branch_rules():
    xs = np.linspace(-12, 12, 50001, dtype=np.float32)
    for x in xs[::7]:
        y = np.float32(orc.gelu_scalar(float(x)))
        if x <= -10:
            assert y == 0
        elif x >= 10:
            assert y == x
        else:
            assert np.float32(y.astype(np.float16)) == y
            # close to the exact tanh-approximated GELU of the f16-rounded input
            q = float(np.float32(x).astype(np.float16))
            ref = 0.5 * q * (1 + math.tanh(0.7978846 * (q + 0.044715 * q ** 3)))
            assert abs(y - ref) <= 2e-3 * max(abs(ref), 1e-2) + 1e-7


def test_rms_norm_closed_form():
    cols, rows = 257, 9
    x = normal(11, cols * rows, 3.0)
    out = np.zeros_like(x)
    assert orc.rms_norm(orc.view(x, [cols, rows, 1, 1]), orc.view(out, [cols, rows, 1, 1]), 1e-6) == orc.OK
    xr = x.reshape(rows, cols).astype(np.float64)
    want = xr / np.sqrt((xr ** 2).mean(axis=1, keepdims=True) + 1e-6)
    assert np.allclose(out.reshape(rows, cols), want, rtol=1e-6, atol=0)
    assert np.allclose(np.sqrt((out.reshape(rows, cols).astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-5)


def test_norm_closed_form():
    cols, rows = 100, 4
    x = normal(12, cols * rows, 2.0) + np.float32(5.0)
    out = np.zeros_like(x)
    assert orc.norm(orc.view(x, [cols, rows, 1, 1]), orc.view(out, [cols, rows, 1, 1]), 1e-6) == orc.OK
    xr = x.reshape(rows, cols).astype(np.float64)
    want = (xr - xr.mean(1, keepdims=True)) / np.sqrt(xr.var(1, keepdims=True) + 1e-6)
    assert np.allclose(out.reshape(rows, cols), want, rtol=1e-5, atol=1e-6)


def test_soft_max_closed_form_and_layouts():
    cols, rows = 300, 7
    x = normal(13, cols * rows, 3.0)
    out = np.zeros_like(x)
    assert orc.soft_max(orc.view(x, [cols, rows, 1, 1]), orc.view(out, [cols, rows, 1, 1])) == orc.OK
    xr = x.reshape(rows, cols).astype(np.float64)
    e = np.exp(xr - xr.max(1, keepdims=True))
    want = e / e.sum(1, keepdims=True)
    # f32 rounding of x - max alone moves exp() by up to |x - max| * 2^-24
    # relatively; |x - max| < 40 here, plus a few ulps from expf and the divide.
    assert np.allclose(out.reshape(rows, cols), want, rtol=4e-6, atol=0)
    assert np.abs(out.reshape(rows, cols).astype(np.float64).sum(1) - 1).max() < 1e-6
    # strided (f32 sequential sum) path: same closed form within f32 summation error
    buf = np.zeros(2 * cols * rows, np.float32)
    buf[::2] = x
    out2 = np.zeros(2 * cols * rows, np.float32)
    nb = [8, 8 * cols, 8 * cols * rows, 8 * cols * rows]
    assert orc.soft_max(orc.view(buf, [cols, rows, 1, 1], nb), orc.view(out2, [cols, rows, 1, 1], nb)) == orc.OK
    assert np.allclose(out2[::2].reshape(rows, cols), want, rtol=1e-5, atol=0)


def test_soft_max_ext_special_cases():
    nkv, nq, nh = 64, 8, 3
    x = normal(14, nkv * nq * nh, 2.0)
    zero = np.zeros(nkv * nq, np.uint16)
    a = np.zeros_like(x)
    b = np.zeros_like(x)
    assert orc.soft_max_ext(orc.view(x, [nkv, nq, nh, 1]), orc.view(zero, [nkv, nq, 1, 1], None, orc.F16), 1.0,
                            orc.view(a, [nkv, nq, nh, 1])) == orc.OK
    assert orc.soft_max(orc.view(x, [nkv, nq, nh, 1]), orc.view(b, [nkv, nq, nh, 1])) == orc.OK
    assert (bits(a) == bits(b)).all()
    # causal mask: masked columns are exactly zero; the rest is softmax of x*scale
    k = np.arange(nkv)[None, :]
    q = np.arange(nq)[:, None]
    allowed = k <= q + (nkv - nq)
    mask = np.where(allowed, np.float16(0), np.float16(-np.inf)).astype(np.float16).view(np.uint16).reshape(-1)
    s = 0.25
    assert orc.soft_max_ext(orc.view(x, [nkv, nq, nh, 1]), orc.view(mask, [nkv, nq, 1, 1], None, orc.F16), s,
                            orc.view(a, [nkv, nq, nh, 1])) == orc.OK
    ar = a.reshape(nh, nq, nkv)
    assert (ar[:, ~allowed] == 0).all()
    xs = (x.reshape(nh, nq, nkv) * np.float32(s)).astype(np.float64)
    xs = np.where(allowed[None], xs, -np.inf)
    e = np.exp(xs - xs.max(-1, keepdims=True))
    assert np.allclose(ar, e / e.sum(-1, keepdims=True), rtol=4e-6, atol=0)


def test_argmax_matches_numpy_first_occurrence():
    g = np.random.Generator(np.random.PCG64(15))
    for trial in range(50):
        n = int(g.integers(1, 300))
        x = g.integers(-5, 5, n).astype(np.float32)  # many ties
        dst = np.zeros(1, np.float32)
        assert orc.argmax(orc.view(x, [n, 1, 1, 1]), orc.view(dst, [1, 1, 1, 1])) == orc.OK
        assert dst[0] == np.argmax(x)
    rows = np.array([[np.nan, 1, 2], [0, np.nan, -1], [-np.inf, -np.inf, -np.inf], [-0.0, 0.0, -0.0]], np.float32)
    out = np.zeros(4, np.int32)
    assert orc.argmax_rows(orc.view(rows.reshape(-1), [3, 4, 1, 1]), orc.view(out, [1, 4, 1, 1])) == orc.OK
    assert list(out) == [0, 0, 0, 0]


def test_sum_rows_close_to_exact_sum():
    cols, rows = 5000, 6
    x = normal(16, cols * rows)
    out = np.zeros(rows, np.float32)
    assert orc.sum_rows(orc.view(x, [cols, rows, 1, 1]), orc.view(out, [1, rows, 1, 1])) == orc.OK
    for r in range(rows):
        exact = math.fsum(float(v) for v in x[r * cols:(r + 1) * cols])
        assert abs(float(out[r]) - exact) <= abs(np.spacing(np.float32(exact))) * 1.0 + 1e-9
    s = np.zeros(1, np.float32)
    assert orc.mean(orc.view(x, [cols, rows, 1, 1]), orc.view(s, [1, 1, 1, 1])) == orc.OK
    assert abs(float(s[0]) - math.fsum(map(float, x)) / x.size) < 1e-7


def test_swiglu_and_rms_norm_mul_compositions():
    n = 1000
    gate = normal(17, n, 3.0)
    up = normal(18, n)
    out = np.zeros(n, np.float32)
    assert orc.swiglu(orc.view(gate, [n, 1, 1, 1]), orc.view(up, [n, 1, 1, 1]), orc.view(out, [n, 1, 1, 1])) == orc.OK
    silu = np.array([orc.silu_scalar(float(v)) for v in gate], np.float32)
    assert (bits(out) == bits(silu * up)).all()
    # silu close to the exact formula (glibc expf is within 1 ulp)
    exact = gate.astype(np.float64) / (1 + np.exp(-gate.astype(np.float64)))
    assert np.allclose(silu, exact, rtol=3e-7, atol=1e-30)
    cols, rows = 64, 5
    x = normal(19, cols * rows)
    w = uniform(20, cols, 0.5, 1.5)
    a = np.zeros_like(x)
    b = np.zeros_like(x)
    assert orc.rms_norm_mul(orc.view(x, [cols, rows, 1, 1]), orc.view(w, [cols, 1, 1, 1]),
                            orc.view(a, [cols, rows, 1, 1]), 1e-5) == orc.OK
    assert orc.rms_norm(orc.view(x, [cols, rows, 1, 1]), orc.view(b, [cols, rows, 1, 1]), 1e-5) == orc.OK
    assert (bits(a) == bits((b.reshape(rows, cols) * w[None, :]).reshape(-1))).all()
