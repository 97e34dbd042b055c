"""CPU: the oracle's restatement of the 21 typed unary events (unary.rs:72-92,
formulas :472-610) and of reductions::OpLog / OpSin / OpCos (reductions.rs:
45-90, :640-668), pinned by the reference's own known answers
(tests/any/unary_ops.rs:24-127, tests/any/reductions.rs:20-56) and, for the
formulas those tests leave open, by independent float64 closed forms."""
import math

import numpy as np
import pytest

import oracle as orc
from emel_hip.abi import UnarySubOp as U

X4 = np.array([-2.0, -0.5, 0.5, 2.0], np.float32)  # unary_ops.rs:26


def ev(code, x):
    out = np.zeros_like(x)
    assert orc.unary_event(int(code), orc.view(x, [x.size, 1, 1, 1]), orc.view(out, [x.size, 1, 1, 1])) == orc.OK
    return out


@pytest.mark.parametrize("code,want", [
    (U.ABS, [2.0, 0.5, 0.5, 2.0]), (U.SGN, [-1.0, -1.0, 1.0, 1.0]), (U.NEG, [2.0, 0.5, -0.5, -2.0]),
    (U.STEP, [0.0, 0.0, 1.0, 1.0]), (U.RELU, [0.0, 0.0, 0.5, 2.0]), (U.FLOOR, [-2.0, -1.0, 0.0, 2.0]),
    (U.CEIL, [-2.0, 0.0, 1.0, 2.0]), (U.ROUND, [-2.0, -1.0, 1.0, 2.0]), (U.TRUNC, [-2.0, 0.0, 0.0, 2.0]),
])
def test_reference_exact_known_answers(code, want):
    assert (ev(code, X4) == np.array(want, np.float32)).all()


def test_reference_approximate_known_answers():
    assert abs(ev(U.SILU, X4)[2] - 0.31122968) < 1e-6                    # unary_ops.rs:77
    assert abs(ev(U.EXP, X4)[0] - math.exp(-2.0)) < 1e-6                 # :85
    assert abs(ev(U.EXPM1, X4)[2] - math.expm1(0.5)) < 1e-6              # :93
    x = np.array([1.0, 2.0, 4.0], np.float32)                            # reductions.rs:23-56
    out = np.zeros_like(x)
    assert orc.log(orc.view(x, [3, 1, 1, 1]), orc.view(out, [3, 1, 1, 1])) == orc.OK
    assert abs(out[0]) < 1e-6 and abs(out[1] - math.log(2.0)) < 1e-6
    assert orc.sin(orc.view(x, [3, 1, 1, 1]), orc.view(out, [3, 1, 1, 1])) == orc.OK
    assert abs(out[0] - math.sin(1.0)) < 1e-6
    assert orc.cos(orc.view(x, [3, 1, 1, 1]), orc.view(out, [3, 1, 1, 1])) == orc.OK
    assert abs(out[0] - math.cos(1.0)) < 1e-6


def grid(seed, n=200_000):
    g = np.random.Generator(np.random.PCG64(seed))
    return np.concatenate([g.standard_normal(n // 2) * 4, g.uniform(-30, 30, n // 2),
                           [0.0, -0.0, 3.0, -3.0, 2.5, -2.5, 0.5, -0.5, 1e-40, -1e-40]]).astype(np.float32)


def f32ops(x):
    return x.astype(np.float32)


def test_sign_step_rounding_closed_forms():
    x = grid(1)
    assert (ev(U.SGN, x) == np.copysign(np.float32(1.0), x)).all()           # signum: +-0 -> +-1
    assert (ev(U.STEP, x) == (x > 0).astype(np.float32)).all()
    xd = x.astype(np.float64)
    assert (ev(U.FLOOR, x) == np.floor(xd)).all() and (ev(U.CEIL, x) == np.ceil(xd)).all()
    assert (ev(U.TRUNC, x) == np.trunc(xd)).all()
    away = np.sign(xd) * np.floor(np.abs(xd) + 0.5)                         # halfway away from zero
    assert (ev(U.ROUND, x) == away).all()
    nan = np.array([np.nan], np.float32)
    assert np.isnan(ev(U.SGN, nan)).all() and ev(U.STEP, nan)[0] == 0.0


def test_sgn_of_every_nan_is_the_canonical_nan():
    # f32::signum returns f32::NAN (0x7fc00000) for any NaN: negative NaNs,
    # payloads and signalling NaNs included (unary.rs:483 calls signum)
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7FC00123, 0xFFFFFFFF, 0x7F800001, 0xFF800001, 0x7FBFFFFF],
                    np.uint32).view(np.float32)
    assert (ev(U.SGN, nans).view(np.uint32) == 0x7FC00000).all()


def test_hard_activations_closed_forms():
    x = grid(2)
    c = np.clip(f32ops(x + np.float32(3.0)), np.float32(0.0), np.float32(6.0))  # each op rounded to f32
    assert (ev(U.HARDSIGMOID, x) == f32ops(c / np.float32(6.0))).all()
    assert (ev(U.HARDSWISH, x) == f32ops(f32ops(x * c) / np.float32(6.0))).all()
    nan = np.array([np.nan], np.float32)
    assert np.isnan(ev(U.HARDSWISH, nan)).all() and np.isnan(ev(U.HARDSIGMOID, nan)).all()


def test_transcendental_formulas_against_float64():
    x = grid(3)
    xd = x.astype(np.float64)
    # softplus = ln(1 + e^x), two f32-rounded libm results: within a few f32 ulps of the exact value
    sp = ev(U.SOFTPLUS, x).astype(np.float64)
    exact = np.logaddexp(0.0, xd)
    assert (np.abs(sp - exact) <= 4 * np.abs(np.spacing(exact.astype(np.float32))).astype(np.float64)).all()
    # gelu_erf with the Abramowitz-Stegun erf (|error| < 1.5e-7) against the exact erf
    from scipy.special import erf
    ge = ev(U.GELU_ERF, x).astype(np.float64)
    assert (np.abs(ge - 0.5 * xd * (1 + erf(xd / math.sqrt(2)))) <= 2e-6 * np.maximum(1.0, np.abs(xd))).all()
    # gelu_quick = 0.5 x (1 + tanh(0.7978846 x (1 + 0.044715 x^2)))
    gq = ev(U.GELU_QUICK, x).astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(0.7978846 * xd * (1 + 0.044715 * xd * xd)))
    assert (np.abs(gq - ref) <= 2e-6 * np.maximum(1.0, np.abs(xd))).all()
    # expm1, sigmoid (two f32 roundings), tanh (fdlibm tanhf) within 3 ulps of float64
    for code, fn in ((U.EXPM1, np.expm1), (U.SIGMOID, lambda v: 1 / (1 + np.exp(-v))), (U.TANH, np.tanh)):
        got = ev(code, x).astype(np.float64)
        want = fn(xd)
        assert (np.abs(got - want) <= 3 * np.abs(np.spacing(want.astype(np.float32))).astype(np.float64) + 1e-45).all(), code


def test_log_sin_cos_against_float64():
    g = np.random.Generator(np.random.PCG64(4))
    x = np.concatenate([g.uniform(0, 1e6, 100_000), g.standard_normal(100_000) * 10, [1e30, -1e30, 3e38]]).astype(np.float32)
    xd = x.astype(np.float64)
    for fn, ref in ((orc.sin, np.sin), (orc.cos, np.cos)):
        out = np.zeros_like(x)
        assert fn(orc.view(x, [x.size, 1, 1, 1]), orc.view(out, [x.size, 1, 1, 1])) == orc.OK
        want = ref(xd)
        assert (np.abs(out - want) <= np.abs(np.spacing(want.astype(np.float32))).astype(np.float64) + 1e-45).all()
    pos = np.abs(x[np.abs(x) > 0])
    out = np.zeros_like(pos)
    assert orc.log(orc.view(pos, [pos.size, 1, 1, 1]), orc.view(out, [pos.size, 1, 1, 1])) == orc.OK
    want = np.log(pos.astype(np.float64))
    assert (np.abs(out - want) <= np.abs(np.spacing(np.abs(want).astype(np.float32))).astype(np.float64)).all()
    sp = np.array([0.0, -0.0, -1.0, np.inf, -np.inf, np.nan], np.float32)
    out = np.zeros_like(sp)
    assert orc.log(orc.view(sp, [6, 1, 1, 1]), orc.view(out, [6, 1, 1, 1])) == orc.OK
    assert out[0] == -np.inf and out[1] == -np.inf and np.isnan(out[2]) and out[3] == np.inf and np.isnan(out[4])
    assert orc.sin(orc.view(sp, [6, 1, 1, 1]), orc.view(out, [6, 1, 1, 1])) == orc.OK
    assert out[0] == 0.0 and np.signbit(out[1]) and np.isnan(out[3]) and np.isnan(out[4])


def test_guards():
    x = np.ones(4, np.float32)
    out = np.full(4, 9.0, np.float32)
    assert orc.unary_event(int(U.XIELU), orc.view(x, [4, 1, 1, 1]), orc.view(out, [4, 1, 1, 1])) == orc.UNEXPECTED_EVENT
    assert orc.unary_event(int(U.SOFTPLUS), orc.view(x, [4, 1, 1, 1]), orc.view(out, [3, 1, 1, 1])) == orc.SHAPE_MISMATCH
    assert orc.log(orc.view(x, [4, 1, 1, 1]), orc.view(out, [2, 1, 1, 1])) == orc.SHAPE_MISMATCH
    assert orc.sin(orc.view(x, [2, 2, 1, 1]), orc.view(out, [4, 1, 1, 1])) == orc.OK  # equal counts, shapes may differ
    assert orc.cos(orc.view(x, [4, 1, 1, 1], [4, 4, 4, 4], data_bytes=8), orc.view(out, [4, 1, 1, 1])) == orc.INVALID_VIEW


def test_relu_ignores_every_nan_as_rust_max_does():
    # Rust documents f32::max / f32::min: "If one of the arguments is NaN, then
    # the other argument is returned" -- signaling NaN included (glibc fmaxf
    # would return a quieted NaN for one)
    nans = np.array([0x7fc00000, 0x7f800001, 0x7fa00025, 0xffc00000, 0xff800001], np.uint32).view(np.float32)
    assert (ev(U.RELU, nans) == 0.0).all()
    # SwiGLU-OAI clamps values and gates with f32::min(x, 7): NaN -> 7
    out = np.zeros(nans.size, np.float32)
    assert orc.glu(orc.SWIGLU_OAI, np.concatenate([nans, nans]), out) == orc.OK
    sevens = np.full(nans.size, 7.0, np.float32)
    want = np.zeros(nans.size, np.float32)
    assert orc.glu(orc.SWIGLU_OAI, np.concatenate([sevens, sevens]), want) == orc.OK
    assert (out == want).all() and np.isfinite(out).all()
