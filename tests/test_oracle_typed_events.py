"""CPU: the oracle's restatement of the typed events of activation.rs,
elementwise.rs, diag.rs and group_norm.rs, pinned by the reference's known
answers (tests/any/activation_ops.rs, elementwise_ops.rs, group_norm_ops.rs,
diag.rs's unit tests) and by numpy closed forms."""
import math

import numpy as np

import oracle as orc


def v(a, ne=None, nb=None, **kw):
    return orc.view(a, ne or [a.size, 1, 1, 1], nb, **kw)


def test_activation_known_answers():
    src = np.array([-2.0, -0.5, 0.0, 2.0], np.float32)                     # activation_ops.rs:22
    out = np.zeros(4, np.float32)
    assert orc.clamp(v(src), v(out), -1.0, 1.0) == orc.OK
    assert (out == np.array([-1.0, -0.5, 0.0, 1.0], np.float32)).all()
    assert orc.leaky_relu(v(src), v(out), 0.1) == orc.OK
    assert (out == np.array([-0.2, -0.05, 0.0, 2.0], np.float32)).all()
    nan = np.array([np.nan], np.float32)
    o1 = np.zeros(1, np.float32)
    assert orc.clamp(v(nan), v(o1), -1.0, 1.0) == orc.OK and np.isnan(o1[0])  # :60-76
    x = np.array([-1.0, 0.0, 1.0], np.float32)                              # :79-97
    g = np.full(3, 2.0, np.float32)
    o3 = np.zeros(3, np.float32)
    assert orc.silu_back(v(x), v(g), v(o3)) == orc.OK
    for i, val in enumerate(x.astype(np.float64)):
        s = 1 / (1 + math.exp(-val))
        assert abs(o3[i] - 2 * s * (val * (1 - s) + 1)) < 1e-6


def test_clamp_is_std_clamp_order():
    # min > max: below min gives min (std::clamp's first comparison), else max
    x = np.array([-5.0, 0.0, 5.0], np.float32)
    out = np.zeros(3, np.float32)
    assert orc.clamp(v(x), v(out), 1.0, -1.0) == orc.OK
    assert (out == np.array([1.0, 1.0, -1.0], np.float32)).all()


def test_elementwise_known_answers():
    x = np.array([1.0, -2.0, 3.5, 4.0], np.float32)                         # elementwise_ops.rs:18-34
    out = np.zeros(4, np.float32)
    assert orc.add1(v(x), 2.0, v(out)) == orc.OK and (out == [3.0, 0.0, 5.5, 6.0]).all()
    base = np.array([1, 2, 3, 4, 5, 6], np.float32)                         # :37-55
    upd = np.array([10, 20], np.float32)
    o6 = np.zeros(6, np.float32)
    assert orc.acc(v(base), v(upd), v(o6), 2) == orc.OK and (o6 == [1, 2, 13, 24, 5, 6]).all()
    o4 = np.full(4, 9.0, np.float32)                                        # :58-86
    assert orc.acc(v(base[:4]), v(upd), v(o4), 3) == orc.INVALID_OFFSET and (o4 == 9.0).all()
    assert orc.add1(v(base[:4]), 1.0, v(o4[:2])) == orc.SHAPE_MISMATCH
    # outside the update the base is copied bit for bit (no +0.0: -0.0 survives)
    nz = np.array([-0.0, -0.0, -0.0], np.float32)
    o = np.zeros(3, np.float32)
    assert orc.acc(v(nz), v(np.array([0.0], np.float32)), v(o), 1) == orc.OK
    assert np.signbit(o[0]) and not np.signbit(o[1]) and np.signbit(o[2])
    # strided (non-dense) views are invalid for acc
    assert orc.acc(v(base, [3, 1, 1, 1], [8, 24, 24, 24]), v(upd), v(o), 0) == orc.INVALID_VIEW


def test_diag_family_known_answers():
    out = np.full(4, 9.0, np.float32)                                       # diag.rs:392-404
    assert orc.diag(np.array([1.0, 2.0], np.float32), out) == orc.OK and (out == [1, 0, 0, 2]).all()
    m = np.zeros(4, np.float32)                                             # :407-419
    assert orc.diag_mask(True, np.array([1, 2, 3, 4], np.float32), m, 0) == orc.OK
    assert m[0] == 1 and m[1] == -np.inf and m[2] == 3 and m[3] == 4
    bad = np.full(3, 7.0, np.float32)                                       # :421-432
    assert orc.diag(np.array([1.0, 2.0], np.float32), bad) == orc.INVALID_SHAPE and (bad == 7).all()
    keep = np.full(4, 8.0, np.float32)                                      # :434-446
    assert orc.diag_mask(False, np.array([1, 2, 3, 4], np.float32), keep, -1) == orc.INVALID_SHAPE
    # closed form: triu(k = 1 + n_past) masked
    g = np.random.Generator(np.random.PCG64(1))
    n, past = 37, 5
    x = g.standard_normal(n * n).astype(np.float32)
    out = np.zeros_like(x)
    assert orc.diag_mask(False, x, out, past) == orc.OK
    want = x.reshape(n, n).copy()
    want[np.triu_indices(n, 1 + past)] = 0.0
    assert (out == want.reshape(-1)).all()


def test_group_norm_known_answers_and_closed_form():
    x = np.array([1, 3, 1, 3, 10, 14, 10, 14], np.float32)                  # group_norm_ops.rs:14-31
    out = np.zeros(8, np.float32)
    assert orc.group_norm(v(x, [2, 1, 4, 1]), v(out, [2, 1, 4, 1]), 2, 0.0) == orc.OK
    assert (out == [-1, 1, -1, 1, -1, 1, -1, 1]).all()
    o4 = np.full(4, 7.0, np.float32)                                        # :58-86
    x4 = np.array([1, 2, 3, 4], np.float32)
    assert orc.group_norm(v(x4, [2, 1, 2, 1]), v(o4, [2, 1, 1, 1]), 1, 0.0) == orc.SHAPE_MISMATCH
    assert orc.group_norm(v(x4, [2, 1, 2, 1]), v(o4, [2, 1, 2, 1]), 3, 0.0) == orc.INVALID_PARAMETERS
    assert (o4 == 7.0).all()
    # closed form: per (batch, group) standardisation in float64
    g = np.random.Generator(np.random.PCG64(2))
    W, H, C, B, G = 5, 3, 12, 2, 4
    x = (g.standard_normal(W * H * C * B) * 3 + 1).astype(np.float32)
    out = np.zeros_like(x)
    assert orc.group_norm(v(x, [W, H, C, B]), v(out, [W, H, C, B]), G, 1e-5) == orc.OK
    xg = x.astype(np.float64).reshape(B, G, -1)
    want = (xg - xg.mean(axis=2, keepdims=True)) / np.sqrt(xg.var(axis=2, keepdims=True) + 1e-5)
    assert np.abs(out.reshape(B, G, -1) - want).max() < 1e-5


def test_l2_norm_known_answers():
    x = np.array([3.0, 4.0, 0.0], np.float32)                               # group_norm_ops.rs:34-56
    out = np.zeros(3, np.float32)
    assert orc.l2_norm(v(x), v(out)) == orc.OK and (out == np.array([0.6, 0.8, 0.0], np.float32)).all()
    z = np.zeros(3, np.float32)
    keep = np.full(3, 5.0, np.float32)
    assert orc.l2_norm(v(z), v(keep)) == orc.ZERO_NORM and (keep == 5.0).all()
    nan = np.array([np.nan, 1.0], np.float32)
    assert orc.l2_norm(v(nan), v(np.zeros(2, np.float32))) == orc.ZERO_NORM  # NaN > 0 is false
