"""GPU parity: the root dense-slice events (event::OpDup / OpAdd / OpSub /
OpMul / OpDiv / OpSqr / OpSqrt over caller slices) and the view power ops
(power::OpSqr / OpSqrt) through the C ABI, vs the CPU oracle, bit-exact
(any NaN matches any NaN); the reference's power manifest cases; the root
InvalidShape rejections leaving the output untouched.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import emel_hip as eh
import oracle as orc
from helpers import Pair, assert_bits_equal, bits, normal, uniform

pytestmark = pytest.mark.gpu

FX = json.loads((Path(__file__).parent / "golden" / "parity_vectors.json").read_text())
BIN = {orc.ADD: eh.DenseOpAdd, orc.SUB: eh.DenseOpSub, orc.MUL: eh.DenseOpMul, orc.DIV: eh.DenseOpDiv}


def specials():
    return np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.1754942e-38, 3.4028235e38, -3.4028235e38,
                     1.0, -1.0, 2.0, 0.5, 1e19, 1e-19, 1.8446743e19], np.float32)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 4097, 11008 * 512])
def test_dup(gpu, n):
    x = normal(500 + n, n)
    x[: min(n, 17)] = specials()[: min(n, 17)]
    d_in, d_out = dev(x), torch.zeros(n, dtype=torch.float32, device=gpu)
    assert eh.Kernel().process_event(eh.DenseOpDup(d_in, d_out)) == eh.Status.OK
    assert np.array_equal(d_out.cpu().numpy().view(np.uint32), x.view(np.uint32))  # bits, NaN payloads too


@pytest.mark.parametrize("op", [orc.ADD, orc.SUB, orc.MUL, orc.DIV])
@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 4097, 11008 * 512])
def test_binary_slices(gpu, op, n):
    a, b = uniform(510 + n, n, -4, 4), uniform(520 + n, n, -4, 4)
    s = specials()
    if n >= s.size * s.size:
        a[: s.size * s.size] = np.repeat(s, s.size)
        b[: s.size * s.size] = np.tile(s, s.size)
    want = np.zeros(n, np.float32)
    assert orc.slice_binary(op, a, b, want) == orc.OK
    d_out = torch.zeros(n, dtype=torch.float32, device=gpu)
    assert eh.Kernel().process_event(BIN[op](dev(a), dev(b), d_out)) == eh.Status.OK
    assert_bits_equal(d_out.cpu().numpy(), want, f"slice op {op}")


@pytest.mark.parametrize("sqrt_", [False, True])
@pytest.mark.parametrize("n", [1, 5, 4097, 11008 * 512])
def test_power_slices(gpu, sqrt_, n):
    x = normal(530 + n, n, 1e3)
    if n >= 17:
        x[:17] = specials()
    want = np.zeros(n, np.float32)
    assert orc.slice_power(sqrt_, x, want) == orc.OK
    d_out = torch.zeros(n, dtype=torch.float32, device=gpu)
    ev = eh.DenseOpSqrt if sqrt_ else eh.DenseOpSqr
    assert eh.Kernel().process_event(ev(dev(x), d_out)) == eh.Status.OK
    assert_bits_equal(d_out.cpu().numpy(), want, "slice power")


@pytest.mark.parametrize("sqrt_", [False, True])
def test_power_views_strided(gpu, sqrt_):
    """Permuted source, dense destination of another shape (ordinal pairing)."""
    ne = [64, 8, 4, 2]
    x = np.abs(normal(540, int(np.prod(ne)), 10.0)) if sqrt_ else normal(540, int(np.prod(ne)), 10.0)
    src = Pair(x, [64, 8, 4, 2], [4, 1024, 256, 8192])  # storage [64, 4, 8, 2] with dims 1 and 2 swapped
    out = Pair(np.zeros(int(np.prod(ne)), np.float32), [512, 8, 1, 1])
    for p in (src, out):
        p.to(gpu)
    ev = eh.OpSqrt if sqrt_ else eh.OpSqr
    assert eh.Kernel().process_event(ev(src.pview(), out.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = out.host.copy()
    assert orc.op_power(sqrt_, src.oview(), orc.view(want, out.ne, out.nb)) == orc.OK
    assert_bits_equal(out.result(), want, "view power")


@pytest.mark.parametrize("case", FX["power"]["cases"], ids=lambda c: c["name"])
def test_power_manifest_on_gpu(gpu, case):
    inp = np.array(case["input"], np.float32)
    d_out = torch.full((case["out_len"],), case["out_fill"], dtype=torch.float32, device=gpu)
    k = eh.Kernel()
    if case["route"] == "view_sqr":
        lay = eh.Layout(eh.DType.F32, case["ne"], case["nb"])
        st = k.process_event(eh.OpSqr(eh.TensorView(dev(inp), lay), eh.TensorViewMut(d_out, lay)))
        host = d_out.cpu().numpy()
        nb = case["nb"] if case["nb"][0] else [4, 4 * case["ne"][0], 0, 0]
        got = np.array([host[(k_ * nb[0]) // 4] for k_ in range(case["ne"][0])], np.float32)
    else:
        ev = eh.DenseOpSqrt if case["route"] == "slice_sqrt" else eh.DenseOpSqr
        st = k.process_event(ev(dev(inp), d_out))
        got = d_out.cpu().numpy()
    assert (st == eh.Status.OK) == (case["status"] == "ok")
    if case["status"] != "ok":
        assert st == eh.Status.INVALID_SHAPE
    assert list(bits(got)) == case["output_bits"]


def test_slice_rejections_leave_output_untouched(gpu):
    k = eh.Kernel()
    a = torch.ones(4, dtype=torch.float32, device=gpu)
    out = torch.full((4,), 9.0, dtype=torch.float32, device=gpu)
    cases = [
        eh.DenseOpDup(a, out, input_len=4, output_len=3),
        eh.DenseOpDup(a, out, input_len=0, output_len=0),
        eh.DenseOpAdd(a, a, out, lhs_len=4, rhs_len=3, output_len=4),
        eh.DenseOpSub(a, a, out, lhs_len=0, rhs_len=0, output_len=0),
        eh.DenseOpMul(a, a, out, lhs_len=4, rhs_len=4, output_len=3),
        eh.DenseOpDiv(a, a, out, lhs_len=3, rhs_len=4, output_len=4),
        eh.DenseOpSqr(a, out, input_len=4, output_len=3),
        eh.DenseOpSqrt(a, out, input_len=0, output_len=4),
    ]
    for ev in cases:
        assert k.process_event(ev) == eh.Status.INVALID_SHAPE, ev
        assert torch.equal(out.cpu(), torch.full((4,), 9.0))
    # partial overlap of output and input is refused; exact aliasing is fine
    assert k.process_event(eh.DenseOpDup(a[:3], a[1:])) == eh.Status.INVALID_ARGUMENT
    assert k.process_event(eh.DenseOpAdd(a, a, a)) == eh.Status.OK
    assert torch.equal(a.cpu(), torch.full((4,), 2.0))
