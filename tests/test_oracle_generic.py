"""CPU: pins the oracle's restatement of the generic wire envelope
(oracle/emel_oracle_generic.c) against the reference's known answers
(crates/emel-kernels/tests/any/generic_envelope.rs), its guard
classification, closed forms, and the typed ops the oracle already pins."""
import math
import struct

import numpy as np
import pytest

import oracle as orc
from helpers import assert_bits_equal, normal, rng, ulp_distance, uniform

# KernelOperation codes (generic.rs:24-337)
DUP, ADD, ADD1, SUB, MUL, DIV, SQR, SQRT, LOG, SIN, COS = 0, 1, 3, 5, 6, 7, 8, 9, 10, 11, 12
SUM, SUM_ROWS, CUMSUM, MEAN, ARGMAX, COUNT_EQUAL, REPEAT, REPEAT_BACK, CONCAT = 13, 14, 15, 16, 17, 18, 19, 20, 21
SILU_BACK, NORM, RMS_NORM, RMS_NORM_BACK, L2_NORM, MUL_MAT, MUL_MAT_ARGMAX = 22, 23, 24, 25, 27, 28, 29
SCALE, GET_ROWS, DIAG, DIAG_MASK_INF, DIAG_MASK_ZERO, SOFT_MAX, SOFT_MAX_BACK = 32, 40, 43, 44, 45, 46, 47
CLAMP, ARANGE, LEAKY_RELU, FILL, UNARY, GLU = 50, 66, 70, 72, 85, 94
U_ABS, U_NEG, U_TANH, U_ELU, U_RELU, U_SIGMOID, U_GELU, U_SILU, U_EXP = 0, 2, 4, 5, 6, 7, 8, 10, 13


def f32p(*vals):
    return b"".join(struct.pack("=f", v) for v in vals)


def i32p(*vals):
    return b"".join(struct.pack("=i", v) for v in vals)


def v(arr, ne, nb=None, dtype=None, data_bytes=None):
    return orc.view(arr, ne, nb, dtype, data_bytes)


def dense(ne):
    nb = [4]
    for d in range(1, 4):
        nb.append(nb[-1] * ne[d - 1])
    return nb


# ---- the reference's known answers (tests/any/generic_envelope.rs) ----------------


def test_reference_known_answers():
    lay = dict(ne=[4, 1, 1, 1], nb=[4, 16, 64, 256])
    a = np.array([1, -2, 3, 4], np.float32)
    b = np.array([2, 4, 6, 8], np.float32)
    d = np.zeros(4, np.float32)
    assert orc.generic(ADD, v(a, **lay), v(b, **lay), None, v(d, **lay), i32p(0)) == orc.OK
    assert d.tolist() == [3, 2, 9, 12]
    d = np.zeros(4, np.float32)
    assert orc.generic(UNARY, v(a, **lay), None, None, v(d, **lay), unary=U_ABS) == orc.OK
    assert d.tolist() == [1, 2, 3, 4]

    x = np.array([1, 2, 3, 4], np.float32)
    l22 = dict(ne=[2, 2, 1, 1], nb=[4, 8, 16, 16])
    y = np.zeros(4, np.float32)
    assert orc.generic(SOFT_MAX, v(x, **l22), None, None, v(y, **l22)) == orc.OK
    assert np.allclose(y, [0.26894143, 0.7310586, 0.26894143, 0.7310586], atol=1e-6, rtol=0)
    y = np.zeros(4, np.float32)
    assert orc.generic(RMS_NORM, v(x, **l22), None, None, v(y, **l22), f32p(1e-5)) == orc.OK
    scale = 1.0 / math.sqrt(2.5 + float(np.float32(1e-5)))
    assert abs(y[0] - scale) < 1e-6 and abs(y[1] - 2 * scale) < 1e-6

    # F16 matmul
    lhs = np.array([0x3C00, 0x4000, 0x4200, 0x4400], np.uint16)
    rhs = np.array([0x4500, 0x4600, 0x4700, 0x4800], np.uint16)
    d = np.zeros(4, np.float32)
    st = orc.generic(MUL_MAT, v(lhs, [2, 2, 1, 1], [2, 4, 8, 8], orc.F16), v(rhs, [2, 2, 1, 1], [2, 4, 8, 8], orc.F16),
                     None, v(d, [2, 2, 1, 1], [4, 8, 16, 16]))
    assert st == orc.OK and d.tolist() == [17, 39, 23, 53]

    # add1, clamp, fill, arange
    s = np.array([1, -2, 3], np.float32)
    l3 = dict(ne=[3, 1, 1, 1], nb=dense([3, 1, 1, 1]))
    d = np.zeros(3, np.float32)
    assert orc.generic(ADD1, v(s, **l3), None, None, v(d, **l3), f32p(2.0)) == orc.OK
    assert d.tolist() == [3, 0, 5]
    assert orc.generic(CLAMP, v(s, **l3), None, None, v(d, **l3), f32p(-1.0, 1.0)) == orc.OK
    assert d.tolist() == [1, -1, 1]
    assert orc.generic(FILL, None, None, None, v(d, **l3), f32p(7.5)) == orc.OK
    assert d.tolist() == [7.5, 7.5, 7.5]
    assert orc.generic(ARANGE, None, None, None, v(d, **l3), f32p(1.5, 0.5)) == orc.OK
    assert d.tolist() == [1.5, 2.0, 2.5]

    # cumsum, diag, diag_mask_inf, concat
    l22d = dict(ne=[2, 2, 1, 1], nb=dense([2, 2, 1, 1]))
    d = np.zeros(4, np.float32)
    assert orc.generic(CUMSUM, v(x, **l22d), None, None, v(d, **l22d)) == orc.OK
    assert d.tolist() == [1, 3, 3, 7]
    ds = np.array([3, 4], np.float32)
    d = np.zeros(4, np.float32)
    assert orc.generic(DIAG, v(ds, [2, 1, 1, 1], dense([2, 1, 1, 1])), None, None, v(d, **l22d)) == orc.OK
    assert d.tolist() == [3, 0, 0, 4]
    d = np.zeros(4, np.float32)
    assert orc.generic(DIAG_MASK_INF, v(x, **l22d), None, None, v(d, **l22d), i32p(0)) == orc.OK
    assert d[0] == 1 and np.isinf(d[1]) and d[2] == 3 and d[3] == 4
    c1, c2, d3 = np.array([1, 2], np.float32), np.array([3], np.float32), np.zeros(3, np.float32)
    st = orc.generic(CONCAT, v(c1, [2, 1, 1, 1], dense([2, 1, 1, 1])), v(c2, [1, 1, 1, 1], dense([1, 1, 1, 1])),
                     None, v(d3, **l3), i32p(0))
    assert st == orc.OK and d3.tolist() == [1, 2, 3]

    # soft_max_back, l2_norm, count_equal
    vals = np.array([0.25, 0.75, 0.5, 0.5], np.float32)
    grads = np.array([1, 2, 3, 4], np.float32)
    d = np.zeros(4, np.float32)
    assert orc.generic(SOFT_MAX_BACK, v(vals, **l22d), v(grads, **l22d), None, v(d, **l22d), i32p(2)) == orc.OK
    assert np.allclose(d, [-0.1875, 0.1875, -0.25, 0.25], atol=1e-6, rtol=0)
    src = np.array([3, 4], np.float32)
    l2 = dict(ne=[2, 1, 1, 1], nb=dense([2, 1, 1, 1]))
    d = np.zeros(2, np.float32)
    assert orc.generic(L2_NORM, v(src, **l2), None, None, v(d, **l2)) == orc.OK
    assert np.allclose(d, [0.6, 0.8], atol=1e-6, rtol=0)
    e = np.zeros(1, np.float32)
    assert orc.generic(COUNT_EQUAL, v(src, **l2), v(src, **l2), None, v(e, [1, 1, 1, 1], dense([1, 1, 1, 1]))) == orc.OK
    assert e[0] == 2.0

    # mul_mat_argmax: rows [1,2], [3,4], [5,6] dotted with [1,1]
    m = np.arange(1, 7, dtype=np.float32)
    ones = np.ones(2, np.float32)
    d = np.zeros(1, np.float32)
    idx = np.full(1, -1, np.int32)
    st = orc.generic(MUL_MAT_ARGMAX, v(m, [2, 3, 1, 1], [4, 8, 24, 24]), v(ones, [2, 1, 1, 1], [4, 8, 8, 8]),
                     None, v(d, [1, 1, 1, 1], [4, 4, 4, 4]), bytes([7] * 3), index_out=idx)
    assert st == orc.OK and abs(d[0] - 11.0) < np.finfo(np.float32).eps and idx[0] == 2


def test_reference_guard_classification():
    # generic_envelope_rejects_bad_span_before_unsupported_outcome
    src = np.zeros(1, np.float32)
    d = np.zeros(1, np.float32)
    lay = dict(ne=[4, 1, 1, 1], nb=[4, 16, 64, 256])
    assert orc.generic(ADD, v(src, **lay), v(src, **lay), v(src, **lay), v(d, **lay)) == orc.INVALID_SHAPE
    # generic_envelope_requires_safe_argmax_destination: validate fails -> InvalidShape
    s16 = np.zeros(4, np.float32)
    d16 = np.zeros(4, np.float32)
    assert orc.generic(MUL_MAT_ARGMAX, v(s16, **lay), v(s16, **lay), v(s16, **lay), v(d16, **lay)) == orc.INVALID_SHAPE
    # an operation with no maintained route and valid views -> UnsupportedOperation
    assert orc.generic(GET_ROWS, v(s16, **lay), None, None, v(d16, **lay)) == orc.UNSUPPORTED_OPERATION
    assert orc.generic(GLU, v(s16, **lay), None, None, v(d16, **lay)) == orc.UNSUPPORTED_OPERATION
    # a maintained operation whose predicate fails -> InvalidShape
    d3 = np.zeros(3, np.float32)
    assert orc.generic(ADD, v(s16, **lay), v(s16, **lay), None, v(d3, [3, 1, 1, 1])) == orc.INVALID_SHAPE
    assert orc.generic(UNARY, v(s16, **lay), None, None, v(d16, **lay), unary=U_SIGMOID) == orc.INVALID_SHAPE
    assert orc.generic(RMS_NORM, v(s16, **lay), None, None, v(d16, **lay), f32p(1e-5), params_size=3) == orc.INVALID_SHAPE
    assert orc.generic(CLAMP, v(s16, **lay), None, None, v(d16, **lay), f32p(1.0, -1.0)) == orc.INVALID_SHAPE
    # unsupported-but-invalid request -> InvalidShape
    assert orc.generic(GET_ROWS, v(src, **lay), None, None, v(d16, **lay)) == orc.INVALID_SHAPE
    # unrepresentable values
    assert orc.generic(95, v(s16, **lay), None, None, v(d16, **lay)) == orc.INVALID_ARGUMENT
    assert orc.generic(ADD, v(s16, **lay), v(s16, **lay), None, v(d16, **lay), params_size=65) == orc.INVALID_ARGUMENT
    # a passed guard with a partial last element: the reference panics
    short = dict(ne=[4, 1, 1, 1], nb=[4, 16, 64, 256], data_bytes=13)
    assert orc.generic(ADD, v(s16, **short), v(s16, **lay), None, v(d16, **lay)) == orc.PANIC


# ---- closed forms and reductions to pinned ops ---------------------------------------


def permuted_src(seed, ne):
    """A float32 view with dims 1 and 2 swapped in memory."""
    buf = normal(seed, int(np.prod(ne)))
    phys = [ne[0], ne[2], ne[1], ne[3]]
    nb_phys = dense(phys)
    nb = [nb_phys[0], nb_phys[2], nb_phys[1], nb_phys[3]]
    logical = buf.reshape(phys[3], phys[2], phys[1], phys[0]).transpose(0, 2, 1, 3)  # [n3, n1, n2, n0] -> logical
    return buf, nb, np.ascontiguousarray(logical).reshape(-1)


@pytest.mark.parametrize("op,fn", [(ADD, np.add), (SUB, np.subtract), (MUL, np.multiply), (DIV, np.divide)])
def test_binary_matches_ieee_float32_through_permuted_views(op, fn):
    ne = [6, 3, 5, 2]
    a, anb, alog = permuted_src(1, ne)
    b = normal(2, 180)
    d = np.zeros(180, np.float32)
    assert orc.generic(op, v(a, ne, anb), v(b, [9, 20, 1, 1]), None, v(d, ne)) == orc.OK
    with np.errstate(all="ignore"):
        assert_bits_equal(d, fn(alog, b), "generic binary")


def test_scalar_family_and_clamp_match_float32():
    x = normal(3, 64) * np.float32(3)
    x[:4] = [np.nan, -0.0, np.inf, -np.inf]
    lay = dict(ne=[8, 8, 1, 1])
    d = np.zeros(64, np.float32)
    assert orc.generic(ADD1, v(x, **lay), None, None, v(d, **lay), f32p(0.75)) == orc.OK
    assert_bits_equal(d, x + np.float32(0.75), "add1")
    assert orc.generic(SCALE, v(x, **lay), None, None, v(d, **lay), f32p(-1.5)) == orc.OK
    assert_bits_equal(d, x * np.float32(-1.5), "scale")
    assert orc.generic(LEAKY_RELU, v(x, **lay), None, None, v(d, **lay), f32p(0.01)) == orc.OK
    with np.errstate(invalid="ignore"):
        assert_bits_equal(d, np.where(x < 0, x * np.float32(0.01), x), "leaky_relu")
    assert orc.generic(CLAMP, v(x, **lay), None, None, v(d, **lay), f32p(-1.0, 2.0)) == orc.OK
    with np.errstate(invalid="ignore"):
        want = np.where(x < -1, np.float32(-1), x)
        want = np.where(want > 2, np.float32(2), want)
    assert_bits_equal(d, want, "clamp")
    assert d[0] != d[0] and np.signbit(d[1])  # NaN passes through; -0 stays -0


def test_unary_routes_equal_the_typed_unary_ops():
    """abs/neg/tanh/elu/relu/silu/exp run the same formulas as OpUnary."""
    x = normal(4, 256) * np.float32(4)
    lay = [16, 16, 1, 1]
    for sub in (U_ABS, U_NEG, U_TANH, U_ELU, U_RELU, U_SILU, U_EXP):
        d = np.zeros(256, np.float32)
        t = np.zeros(256, np.float32)
        assert orc.generic(UNARY, v(x, lay), None, None, v(d, lay), unary=sub) == orc.OK
        assert orc.unary(sub, v(x, lay), v(t, lay)) == orc.OK
        assert_bits_equal(d, t, f"unary {sub}")


def test_generic_gelu_is_the_unrounded_tanh_formula():
    x = np.linspace(-12, 12, 4001).astype(np.float32)
    d = np.zeros_like(x)
    lay = [x.size, 1, 1, 1]
    assert orc.generic(UNARY, v(x, lay), None, None, v(d, lay), unary=U_GELU) == orc.OK
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1.0 + np.tanh(0.7978846 * (xd + 0.044715 * xd ** 3)))
    assert np.all(np.abs(d - want) <= 4e-6 * np.abs(want) + 1e-6)
    # unlike the typed GELU: no saturation at |x| >= 10 and no fp16 rounding
    assert d[-1] == x[-1] and d[0] == 0.0  # exact limits of the formula at +-12
    mid = x[(x > 0.3) & (x < 0.31)][0]
    assert d[x == mid][0] != np.float32(np.float16(d[x == mid][0]))


def test_silu_back_is_the_derivative_of_silu():
    x = np.linspace(-8, 8, 321).astype(np.float32)
    g = np.full_like(x, 1.0)
    d = np.zeros_like(x)
    lay = [x.size, 1, 1, 1]
    assert orc.generic(SILU_BACK, v(x, lay), v(g, lay), None, v(d, lay)) == orc.OK
    xd = x.astype(np.float64)
    h = 1e-4
    silu = lambda t: t / (1 + np.exp(-t))
    fd = (silu(xd + h) - silu(xd - h)) / (2 * h)
    assert np.max(np.abs(d - fd)) < 1e-5
    assert d[x == 0][0] == 0.5
    # the gradient scales the derivative
    g2 = np.full_like(x, 2.0)
    d2 = np.zeros_like(x)
    assert orc.generic(SILU_BACK, v(x, lay), v(g2, lay), None, v(d2, lay)) == orc.OK
    assert_bits_equal(d2, d * 2, "silu_back gradient scale")


def test_reductions_equal_the_typed_reductions():
    x = normal(5, 4 * 7 * 3)
    ne = [4, 7, 3, 1]
    scal = dict(ne=[1, 1, 1, 1])
    for op, fn in ((SUM, orc.sum_), (MEAN, orc.mean), (ARGMAX, orc.argmax)):
        d, t = np.zeros(1, np.float32), np.zeros(1, np.float32)
        assert orc.generic(op, v(x, ne), None, None, v(d, **scal)) == orc.OK
        assert fn(v(x, ne), v(t, **scal)) == orc.OK
        assert_bits_equal(d, t, f"reduction {op}")


def test_power_and_log_family():
    x = np.abs(normal(6, 50)) + np.float32(0.01)
    lay = [50, 1, 1, 1]
    d = np.zeros(50, np.float32)
    assert orc.generic(SQR, v(x, lay), None, None, v(d, lay)) == orc.OK
    assert_bits_equal(d, x * x, "sqr")
    assert orc.generic(SQRT, v(x, lay), None, None, v(d, lay)) == orc.OK
    assert_bits_equal(d, np.sqrt(x), "sqrt")
    for op, fn in ((LOG, np.log), (SIN, np.sin), (COS, np.cos)):
        assert orc.generic(op, v(x, lay), None, None, v(d, lay)) == orc.OK
        assert np.all(ulp_distance(d, fn(x.astype(np.float64)).astype(np.float32)) <= 1)


def test_softmax_equals_the_typed_strided_softmax():
    """The generic softmax and OpSoftMax's strided path both keep an f32
    running sum; on strided views (the typed op's f32 path) they agree."""
    ne = [33, 4, 3, 1]
    a, nb, _ = permuted_src(7, ne)
    d, t = np.zeros(a.size, np.float32), np.zeros(a.size, np.float32)
    assert orc.generic(SOFT_MAX, v(a, ne, nb), None, None, v(d, ne)) == orc.OK
    assert orc.soft_max(v(a, ne, nb), v(t, ne)) == orc.OK
    assert_bits_equal(d, t, "generic vs typed strided softmax")
    rows = d.reshape(-1, 33).astype(np.float64).sum(axis=1)
    assert np.all(np.abs(rows - 1) < 1e-5)


def test_softmax_skips_nan_in_the_maximum():
    x = np.array([np.nan, 1.0, 2.0, 3.0], np.float32)
    d = np.zeros(4, np.float32)
    assert orc.generic(SOFT_MAX, v(x, [4, 1, 1, 1]), None, None, v(d, [4, 1, 1, 1])) == orc.OK
    assert np.isnan(d).all()  # exp(NaN) poisons the sum; the maximum came from the finite values


def test_norms_track_the_typed_norms():
    """The generic norms compute their scale in f64; the typed ones in f32.
    Both are pinned formulas of the same quantity: within 2 ulp."""
    ne = [64, 9, 2, 1]
    x = normal(8, int(np.prod(ne))) * np.float32(3)
    for op, fn in ((RMS_NORM, orc.rms_norm), (NORM, orc.norm)):
        d, t = np.zeros(x.size, np.float32), np.zeros(x.size, np.float32)
        assert orc.generic(op, v(x, ne), None, None, v(d, ne), f32p(1e-5)) == orc.OK
        assert fn(v(x, ne), v(t, ne), 1e-5) == orc.OK
        assert np.max(ulp_distance(d, t)) <= 2, op


def test_cumsum_is_numpys_sequential_float32_cumsum():
    ne = [37, 5, 2, 1]
    a, nb, alog = permuted_src(9, ne)
    d = np.zeros(a.size, np.float32)
    assert orc.generic(CUMSUM, v(a, ne, nb), None, None, v(d, ne)) == orc.OK
    want = np.cumsum(alog.reshape(-1, 37), axis=1, dtype=np.float32).reshape(-1)
    assert_bits_equal(d, want, "cumsum")


def test_repeat_and_repeat_back():
    src = rng(10).integers(-8, 8, 3 * 2 * 1 * 2).astype(np.float32)
    sne, tne = [3, 2, 1, 2], [6, 4, 3, 2]
    rep = np.zeros(int(np.prod(tne)), np.float32)
    assert orc.generic(REPEAT, v(src, sne), None, None, v(rep, tne)) == orc.OK
    s4 = src.reshape(2, 1, 2, 3)
    assert_bits_equal(rep, np.tile(s4, (1, 3, 2, 2)).reshape(-1), "repeat")
    back = np.zeros(src.size, np.float32)
    assert orc.generic(REPEAT_BACK, v(rep, tne), None, None, v(back, sne)) == orc.OK
    assert_bits_equal(back, src * np.float32(2 * 2 * 3), "repeat_back of repeat")


def test_concat_diag_and_masks():
    g = rng(11)
    for axis in range(4):
        lne = [2, 3, 2, 2]
        rne = list(lne)
        rne[axis] = 3
        dne = list(lne)
        dne[axis] += 3
        lhs = g.standard_normal(int(np.prod(lne))).astype(np.float32)
        rhs = g.standard_normal(int(np.prod(rne))).astype(np.float32)
        d = np.zeros(int(np.prod(dne)), np.float32)
        assert orc.generic(CONCAT, v(lhs, lne), v(rhs, rne), None, v(d, dne), i32p(axis)) == orc.OK
        want = np.concatenate([lhs.reshape(lne[::-1]), rhs.reshape(rne[::-1])], axis=3 - axis).reshape(-1)
        assert_bits_equal(d, want, f"concat axis {axis}")
        # the axis parameter must name the axis the shapes concatenate along
        assert orc.generic(CONCAT, v(lhs, lne), v(rhs, rne), None, v(d, dne), i32p((axis + 1) % 4)) == orc.INVALID_SHAPE
    s = g.standard_normal(5).astype(np.float32)
    d = np.zeros(25, np.float32)
    assert orc.generic(DIAG, v(s, [5, 1, 1, 1]), None, None, v(d, [5, 5, 1, 1])) == orc.OK
    assert_bits_equal(d, np.diag(s).reshape(-1), "diag")
    x = g.standard_normal(36).astype(np.float32)
    for n_past in (0, 2, 7):
        for op, fill in ((DIAG_MASK_INF, -np.inf), (DIAG_MASK_ZERO, 0.0)):
            d = np.zeros(36, np.float32)
            assert orc.generic(op, v(x, [6, 6, 1, 1]), None, None, v(d, [6, 6, 1, 1]), i32p(n_past)) == orc.OK
            row, col = np.divmod(np.arange(36), 6)
            assert_bits_equal(d, np.where(col > row + n_past, np.float32(fill), x), f"mask {op} {n_past}")


def test_arange_and_fill():
    d = np.zeros(1000, np.float32)
    assert orc.generic(ARANGE, None, None, None, v(d, [10, 100, 1, 1]), f32p(-3.25, 0.125)) == orc.OK
    assert_bits_equal(d, (np.arange(1000) * 0.125 - 3.25).astype(np.float32), "arange")
    assert orc.generic(FILL, None, None, None, v(d, [10, 100, 1, 1]), f32p(-0.0)) == orc.OK
    assert np.all(np.signbit(d)) and np.all(d == 0)
    # fill and arange take no source
    s = np.zeros(1000, np.float32)
    assert orc.generic(FILL, v(s, [1000, 1, 1, 1]), None, None, v(d, [1000, 1, 1, 1]), f32p(1.0)) == orc.INVALID_SHAPE


def test_l2_norm_and_count_equal():
    x = normal(12, 300)
    d = np.zeros(300, np.float32)
    assert orc.generic(L2_NORM, v(x, [30, 10, 1, 1]), None, None, v(d, [30, 10, 1, 1])) == orc.OK
    assert abs(np.sqrt(np.sum(d.astype(np.float64) ** 2)) - 1) < 1e-5
    y = x.copy()
    y[::3] += 1
    y[5] = np.nan
    x2 = x.copy()
    x2[5] = np.nan  # equal bits count, NaN included
    e = np.zeros(1, np.float32)
    assert orc.generic(COUNT_EQUAL, v(x2, [300, 1, 1, 1]), v(y, [10, 30, 1, 1]), None, v(e, [1, 1, 1, 1])) == orc.OK
    assert e[0] == float(np.sum(x2.view(np.uint32) == y.view(np.uint32)))


def test_count_equal_saturates_like_an_f32_counter():
    n = (1 << 24) + 7
    a = np.zeros(n, np.float32)
    e = np.zeros(1, np.float32)
    assert orc.generic(COUNT_EQUAL, v(a, [n, 1, 1, 1]), v(a, [n, 1, 1, 1]), None, v(e, [1, 1, 1, 1])) == orc.OK
    assert e[0] == float(1 << 24)


def test_softmax_back_and_rms_norm_back():
    ne = [8, 6, 1, 1]
    vals = np.abs(normal(13, 48))
    vals /= vals.reshape(6, 8).sum(axis=1).repeat(8)
    grads = normal(14, 48)
    d = np.zeros(48, np.float32)
    assert orc.generic(SOFT_MAX_BACK, v(vals, ne), v(grads, ne), None, v(d, ne), i32p(8)) == orc.OK
    v64, g64 = vals.reshape(6, 8).astype(np.float64), grads.reshape(6, 8).astype(np.float64)
    want = v64 * (g64 - (v64 * g64).sum(axis=1, keepdims=True))
    assert np.max(np.abs(d.reshape(6, 8) - want)) < 1e-6
    # a constant gradient over a normalised row gives zero
    c = np.full(48, 3.0, np.float32)
    assert orc.generic(SOFT_MAX_BACK, v(vals, ne), v(c, ne), None, v(d, ne), i32p(8)) == orc.OK
    assert np.max(np.abs(d)) < 1e-6
    # rms_norm_back is the gradient of y = x / rms(x) contracted with dy
    x = normal(15, 48)
    dy = normal(16, 48)
    eps = 1e-5
    assert orc.generic(RMS_NORM_BACK, v(x, ne), v(dy, ne), None, v(d, ne), f32p(eps)) == orc.OK

    def loss(xr):
        return np.sum(dy.reshape(6, 8).astype(np.float64) * xr / np.sqrt(np.mean(xr * xr, axis=1, keepdims=True) + float(np.float32(eps))))

    x64 = x.reshape(6, 8).astype(np.float64)
    fd = np.zeros_like(x64)
    h = 1e-6
    for i in range(6):
        for j in range(8):
            p, m = x64.copy(), x64.copy()
            p[i, j] += h
            m[i, j] -= h
            fd[i, j] = (loss(p) - loss(m)) / (2 * h)
    assert np.max(np.abs(d.reshape(6, 8) - fd)) < 1e-4


def test_mul_mat_within_the_fma_chain_bound():
    g = rng(17)
    k, m, n = 37, 5, 7
    lhs = g.standard_normal(k * m).astype(np.float32)
    rhs = g.standard_normal(n * k).astype(np.float32)
    d = np.zeros(n * m, np.float32)
    assert orc.generic(MUL_MAT, v(lhs, [k, m, 1, 1]), v(rhs, [n, k, 1, 1]), None, v(d, [n, m, 1, 1])) == orc.OK
    L = lhs.reshape(m, k).astype(np.float64)
    R = rhs.reshape(k, n).astype(np.float64)
    exact = L @ R
    bound = k * 2.0 ** -24 * (np.abs(L) @ np.abs(R))
    assert np.all(np.abs(d.reshape(m, n) - exact) <= bound)
    # a single-term dot is exact: k = 1 gives the outer product
    o = np.zeros(n * m, np.float32)
    assert orc.generic(MUL_MAT, v(lhs[:m], [1, m, 1, 1]), v(rhs[:n], [n, 1, 1, 1]), None, v(o, [n, m, 1, 1])) == orc.OK
    assert_bits_equal(o, np.outer(lhs[:m], rhs[:n]).astype(np.float32).reshape(-1), "outer")


def test_f16_mul_mat_matches_the_exact_product():
    g = rng(18)
    k, m, n = 40, 6, 3
    lhs = g.standard_normal(k * m).astype(np.float16)
    rhs = g.standard_normal(k * n).astype(np.float16)
    d = np.zeros(m * n, np.float32)
    st = orc.generic(MUL_MAT, v(lhs.view(np.uint16), [k, m, 1, 1], [2, 2 * k, 2 * k * m, 2 * k * m], orc.F16),
                     v(rhs.view(np.uint16), [k, n, 1, 1], [2, 2 * k, 2 * k * n, 2 * k * n], orc.F16), None,
                     v(d, [m, n, 1, 1]))
    assert st == orc.OK
    # f16 x f16 products are exact in f32; their f64 sum rounds once to f32
    exact = (lhs.reshape(m, k).astype(np.float64) @ rhs.reshape(n, k).astype(np.float64).T)  # [m, n]
    got = d.reshape(n, m).T  # dst ordinal row + col * m
    assert np.max(ulp_distance(got, exact.astype(np.float32))) <= 1


def test_mul_mat_argmax_first_row_and_nan_rule():
    k = 3
    ones = np.ones(k, np.float32)
    m = np.array([[1, 1, 1], [2, 2, 2], [2, 2, 2], [0, 0, 0]], np.float32).reshape(-1)
    d = np.zeros(1, np.float32)
    idx = np.zeros(1, np.int32)
    args = lambda mm: (v(mm, [k, 4, 1, 1]), v(ones, [k, 1, 1, 1]), None, v(d, [1, 1, 1, 1]))
    assert orc.generic(MUL_MAT_ARGMAX, *args(m), index_out=idx) == orc.OK
    assert idx[0] == 1 and d[0] == 6.0  # first of the tied rows
    m0 = m.copy()
    m0[0] = np.nan
    assert orc.generic(MUL_MAT_ARGMAX, *args(m0), index_out=idx) == orc.OK
    assert idx[0] == 0 and np.isnan(d[0])  # a NaN in row 0 is never beaten
    m2 = m.copy()
    m2[3 * k] = np.nan  # row 3
    assert orc.generic(MUL_MAT_ARGMAX, *args(m2), index_out=idx) == orc.OK
    assert idx[0] == 1  # later NaNs are skipped
    m3 = m.copy()
    m3[1 * k] = np.nan  # row 1: its tie partner row 2 wins
    assert orc.generic(MUL_MAT_ARGMAX, *args(m3), index_out=idx) == orc.OK
    assert idx[0] == 2 and d[0] == 6.0
