"""CPU: the oracle's OpGlu (glu.rs) pinned by the reference's own unit tests
(glu.rs:295-365) and by checks the formulas fix independently:

  SwiGLU   == the OpSilu -> OpMul composition (an already pinned path), bits;
  ReGLU    == values * (gate > 0 ? gate : 0) in numpy float32, bits;
  GeGLU    == the tanh approximation evaluated in float64, to 2e-6 relative
              (plus the f32 cancellation of 1 + tanh(z) near z = -9);
  GeGLU-erf == 0.5 x (1 + erf(x / sqrt 2)) with the exact erf, to 2e-6
              absolute (Abramowitz-Stegun 7.1.26 is within 1.5e-7);
  GeGLU-quick, SwiGLU-OAI == their formulas in float64, to 2e-6 relative.

No parity manifest in the reference covers GLU, so these are its pins.
"""
import math

import numpy as np
import pytest

import oracle as orc
from helpers import normal

SUBOPS = [orc.REGLU, orc.GEGLU, orc.SWIGLU, orc.SWIGLU_OAI, orc.GEGLU_ERF, orc.GEGLU_QUICK]


def run(subop, values, gates):
    inp = np.concatenate([values, gates]).astype(np.float32)
    out = np.full(values.size, 123.0, np.float32)
    assert orc.glu(subop, inp, out) == orc.OK
    return out


def test_reglu_known_answer():
    """glu.rs reglu_multiplies_relu_gate: [1, -2 | 3, 4] -> [3, -8]."""
    out = np.zeros(2, np.float32)
    assert orc.glu(orc.REGLU, np.array([1, -2, 3, 4], np.float32), out) == orc.OK
    assert out.view(np.uint32).tolist() == np.array([3.0, -8.0], np.float32).view(np.uint32).tolist()


def test_public_reglu_known_answer():
    """glu.rs public_kernel_dispatches_reglu: [1 | 2] -> [2]."""
    out = np.zeros(1, np.float32)
    assert orc.glu(orc.REGLU, np.array([1, 2], np.float32), out) == orc.OK
    assert out[0] == np.float32(2.0)


def test_odd_length_is_rejected_and_untouched():
    """glu.rs odd_length_is_invalid_and_does_not_mutate."""
    out = np.full(1, 9.0, np.float32)
    assert orc.glu(orc.SWIGLU, np.array([1, 2, 3], np.float32), out) == orc.SHAPE_MISMATCH
    assert out[0] == np.float32(9.0)
    assert orc.glu(orc.SWIGLU, np.zeros(0, np.float32), np.zeros(0, np.float32)) == orc.SHAPE_MISMATCH
    assert orc.glu(orc.SWIGLU, np.zeros(4, np.float32), np.zeros(3, np.float32)) == orc.SHAPE_MISMATCH
    assert orc.glu(6, np.zeros(4, np.float32), np.zeros(2, np.float32)) == orc.UNEXPECTED_EVENT


def test_remaining_subops_are_finite_and_written():
    """glu.rs remaining_glu_subops_write_finite_gated_products: [2 | 1]."""
    for sub in (orc.GEGLU, orc.SWIGLU, orc.SWIGLU_OAI, orc.GEGLU_ERF, orc.GEGLU_QUICK):
        out = np.full(1, 9.0, np.float32)
        assert orc.glu(sub, np.array([2, 1], np.float32), out) == orc.OK
        assert np.isfinite(out[0]) and out[0] != np.float32(9.0)


def test_swiglu_equals_silu_then_mul():
    v, g = normal(41, 4097), normal(42, 4097, 3.0)
    got = run(orc.SWIGLU, v, g)
    want = np.zeros_like(v)
    vw = orc.view(want, [v.size, 1, 1, 1])
    assert orc.swiglu(orc.view(g, [g.size, 1, 1, 1]), orc.view(v, [v.size, 1, 1, 1]), vw) == orc.OK
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_reglu_closed_form():
    v, g = normal(43, 5000), normal(44, 5000)
    g[:7] = [0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3e38]
    want = (v * np.where(g > 0, g, np.float32(0))).astype(np.float32)
    got = run(orc.REGLU, v, g)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _close(got, want, tol, scale):
    """Relative tolerance plus an absolute term for the f32 cancellation in
    1 + tanh(z) (tanhf is exactly -1 for z < -9): ~ulp(1) * |v * g|."""
    want = np.asarray(want, np.float64)
    err = np.abs(got.astype(np.float64) - want)
    return np.all(err <= tol * np.abs(want) + 2e-7 * scale)


@pytest.mark.parametrize("sub", [orc.GEGLU, orc.GEGLU_QUICK, orc.SWIGLU_OAI])
def test_formulas_in_float64(sub):
    v, g = normal(45, 3000, 2.0), normal(46, 3000, 3.0)
    got = run(sub, v, g)
    vd, gd = v.astype(np.float64), g.astype(np.float64)
    if sub == orc.GEGLU:
        want = vd * 0.5 * gd * (1 + np.tanh(0.7978846 * gd * (1 + 0.044715 * gd * gd)))
    elif sub == orc.GEGLU_QUICK:
        want = vd * gd / (1 + np.exp(-1.702 * gd))
    else:
        gc, vc = np.minimum(gd, 7.0), np.minimum(vd, 7.0)
        a = 1.702 * gc
        want = a / (1 + np.exp(-a)) / 1.702 * (vc + 1)
    assert _close(got, want, 2e-6, np.abs(vd) * (np.abs(gd) + 1))


def test_gelu_erf_against_exact_erf():
    g = np.concatenate([np.linspace(-8, 8, 4001, dtype=np.float32), np.array([0.0, -0.0], np.float32)])
    for x in g:
        y = orc.glu_gate(orc.GEGLU_ERF, float(x))
        exact = 0.5 * float(x) * (1 + math.erf(float(x) / math.sqrt(2)))
        assert abs(y - exact) <= 2e-6 * max(1.0, abs(float(x))), (x, y, exact)


def test_swiglu_oai_clamps_nan_gate_to_limit():
    """f32::min(NaN, 7) is 7, so a NaN gate behaves as the limit."""
    got = run(orc.SWIGLU_OAI, np.array([1.0], np.float32), np.array([np.nan], np.float32))
    want = run(orc.SWIGLU_OAI, np.array([1.0], np.float32), np.array([7.0], np.float32))
    assert got[0] == want[0]
