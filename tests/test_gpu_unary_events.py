"""GPU parity: the 21 typed unary events (emel_op_unary_event, unary.rs:72-92)
and reductions::OpLog / OpSin / OpCos (emel_op_log/sin/cos), bit-exact
against the oracle.  Inputs: every 256th f32 bit pattern (2^24 values
spread over all exponents and signs, NaN and infinities included) and
targeted values (halfway points for round, arguments near multiples of
pi/2 and beyond the 120 threshold of sin/cos, near 0 and 1 for log);
strided and reshaped views follow the reference's ordinal addressing."""
import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from emel_hip.abi import UnarySubOp as U
from helpers import Pair, assert_bits_equal

pytestmark = pytest.mark.gpu

EVENTS = [c for c in U if c != U.XIELU]
MATH = {"log": (eh.OpLog, orc.log), "sin": (eh.OpSin, orc.sin), "cos": (eh.OpCos, orc.cos)}


def sweep():
    """Every 256th bit pattern plus targeted values."""
    patterns = (np.arange(1 << 24, dtype=np.uint64) * 256 + 37).astype(np.uint32).view(np.float32)
    g = np.random.Generator(np.random.PCG64(501))
    halves = (np.arange(-4000, 4000, dtype=np.float32) + np.float32(0.5))
    near_pio2 = (np.arange(-400, 400, dtype=np.float64) * (np.pi / 2)).astype(np.float32)
    near_pio2 = np.concatenate([near_pio2, np.nextafter(near_pio2, np.float32(np.inf)),
                                np.nextafter(near_pio2, np.float32(-np.inf))])
    special = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 119.99, 120.0, 120.01, -120.0, 1e-40, 3.4e38,
                        -3.4e38, 88.7, -88.7, 10.0, -10.0, 3.0, -3.0], np.float32)
    return np.concatenate([patterns, halves, near_pio2, special, g.standard_normal(1 << 16).astype(np.float32) * 5,
                           g.uniform(0.5, 2.0, 1 << 16).astype(np.float32)])


@pytest.fixture(scope="module")
def xs():
    return sweep()


def run_event(gpu, build, ofn, x, ne, nb=None, one=None):
    a = Pair(x, ne, nb).to(gpu)
    n = int(np.prod(ne))
    o = Pair(np.zeros(n, np.float32), one or [n, 1, 1, 1]).to(gpu)
    assert eh.Kernel().process_event(build(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = np.zeros(n, np.float32)
    assert ofn(a.oview(), orc.view(want, o.ne)) == orc.OK
    return o.result(), want


@pytest.mark.parametrize("code", EVENTS, ids=[c.name for c in EVENTS])
def test_typed_unary_event_bit_exact(gpu, xs, code):
    print(f"unary event {code.name}: {xs.size} values", flush=True)
    got, want = run_event(gpu, lambda i, o: eh.OpUnaryEvent(code, i, o),
                          lambda i, o: orc.unary_event(int(code), i, o), xs, [xs.size, 1, 1, 1])
    assert_bits_equal(got, want, code.name)


def test_sgn_nan_bits(gpu):
    # assert_bits_equal lets any NaN match any NaN; f32::signum's NaN is
    # the one quiet NaN 0x7fc00000, checked bit for bit here
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7FC00123, 0xFFFFFFFF, 0x7F800001, 0xFF800001, 0x7FBFFFFF, 0x3F800000],
                    np.uint32).view(np.float32)
    got, want = run_event(gpu, lambda i, o: eh.OpUnaryEvent(U.SGN, i, o), lambda i, o: orc.unary_event(int(U.SGN), i, o),
                          nans, [nans.size, 1, 1, 1])
    assert (got.view(np.uint32) == want.view(np.uint32)).all(), (got.view(np.uint32), want.view(np.uint32))
    assert (got.view(np.uint32)[:7] == 0x7FC00000).all() and got[7] == 1.0


@pytest.mark.parametrize("name", list(MATH))
def test_log_sin_cos_bit_exact(gpu, xs, name):
    print(f"{name}: {xs.size} values", flush=True)
    cls, ofn = MATH[name]
    got, want = run_event(gpu, cls, ofn, xs, [xs.size, 1, 1, 1])
    assert_bits_equal(got, want, name)


@pytest.mark.parametrize("code", [U.SOFTPLUS, U.ROUND, U.GELU_ERF, U.HARDSWISH])
def test_typed_unary_strided_and_reshaped(gpu, code):
    g = np.random.Generator(np.random.PCG64(502))
    x = (g.standard_normal(2 * 48 * 36) * 6).astype(np.float32)
    # every other float of padded rows, written to a [36, 48] dst: ordinal pairing
    ne, nb = [48, 36, 1, 1], [8, 8 * 48, 8 * 48 * 36, 8 * 48 * 36]
    got, want = run_event(gpu, lambda i, o: eh.OpUnaryEvent(code, i, o), lambda i, o: orc.unary_event(int(code), i, o),
                          x, ne, nb, one=[36, 48, 1, 1])
    assert_bits_equal(got, want, f"{code.name} strided")
    for name, (cls, ofn) in MATH.items():
        got, want = run_event(gpu, cls, ofn, x, ne, nb, one=[36, 48, 1, 1])
        assert_bits_equal(got, want, f"{name} strided")


def test_guards_leave_dst_untouched(gpu):
    x = Pair(np.ones(8, np.float32), [8, 1, 1, 1]).to(gpu)
    o = Pair(np.full(8, 9.0, np.float32), [8, 1, 1, 1]).to(gpu)
    short = Pair(np.full(6, 9.0, np.float32), [6, 1, 1, 1]).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpUnaryEvent(U.XIELU, x.pview(), o.pview(mut=True))) == eh.Status.UNEXPECTED_EVENT
    assert k.process_event(eh.OpUnaryEvent(99, x.pview(), o.pview(mut=True))) == eh.Status.UNEXPECTED_EVENT
    assert k.process_event(eh.OpSoftplus(x.pview(), short.pview(mut=True))) == eh.Status.SHAPE_MISMATCH
    assert k.process_event(eh.OpLog(x.pview(), short.pview(mut=True))) == eh.Status.SHAPE_MISMATCH
    bad = Pair(np.ones(8, np.float32), [8, 1, 1, 1], data_bytes=16).to(gpu)  # span past data_bytes
    assert k.process_event(eh.OpCos(bad.pview(), o.pview(mut=True))) == eh.Status.INVALID_VIEW
    assert (o.result() == 9.0).all() and (short.result() == 9.0).all()
