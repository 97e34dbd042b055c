"""GPU parity: OpGlu (glu.rs) through emel_op_glu vs the CPU oracle,
bit-exact (any NaN matches any NaN), for all six gates: dense float4 paths
(n % 4 == 0), the scalar path (n % 4 != 0: the gates half is not 16-byte
aligned), the config 2 size, special values in both halves, and the
reference's rejections (odd / empty input, wrong output length, unknown
subop) leaving the output untouched.
"""
import numpy as np
import pytest
import torch

import emel_hip as eh
import oracle as orc
from helpers import assert_bits_equal, normal

pytestmark = pytest.mark.gpu

SUBOPS = [eh.GluSubOp.REGLU, eh.GluSubOp.GEGLU, eh.GluSubOp.SWIGLU, eh.GluSubOp.SWIGLU_OAI,
          eh.GluSubOp.GEGLU_ERF, eh.GluSubOp.GEGLU_QUICK]


def specials():
    f = np.float32
    return np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.1754942e-38, 3.4028235e38,
                     -3.4028235e38, 1.0, -1.0, 7.0, np.nextafter(f(7), f(8)), -7.0, 9.0, -9.0, 20.0, -20.0,
                     88.72283, -88.72283, 60.0, -60.0, -104.0, 1e-20, -1e-20], np.float32)


def run(gpu, sub, values, gates):
    inp = np.concatenate([values, gates]).astype(np.float32)
    want = np.zeros(values.size, np.float32)
    assert orc.glu(int(sub), inp, want) == orc.OK
    d_in = torch.from_numpy(inp).to(gpu)
    d_out = torch.full((values.size,), 123.0, dtype=torch.float32, device=gpu)
    st = eh.Kernel().process_event(eh.OpGlu(d_in, d_out, sub))
    assert st == eh.Status.OK, eh.last_error()
    assert_bits_equal(d_out.cpu().numpy(), want, f"glu {sub.name} n={values.size}")


@pytest.mark.parametrize("sub", SUBOPS)
@pytest.mark.parametrize("n", [1, 3, 4, 1000, 1001, 4097])
def test_glu_random(gpu, sub, n):
    run(gpu, sub, normal(100 + n, n, 2.0), normal(200 + n, n, 4.0))


@pytest.mark.parametrize("sub", SUBOPS)
def test_glu_specials(gpu, sub):
    s = specials()
    values = np.repeat(s, s.size)
    gates = np.tile(s, s.size)
    run(gpu, sub, values, gates)


@pytest.mark.parametrize("sub", SUBOPS)
def test_glu_config2_size(gpu, sub):
    """Config 2's SwiGLU chain as one OpGlu: values = up, gates = gate."""
    n = 11008 * 512
    run(gpu, sub, normal(301, n), normal(302, n))


def test_glu_wide_gate_range(gpu):
    """Gates over the whole exp/tanh range, including every branch of the
    replicas (|z| < 2^-12, < 1, < 22, overflow, underflow)."""
    g = np.concatenate([np.linspace(-120, 120, 200001, dtype=np.float32),
                        np.geomspace(1e-30, 1e2, 20000, dtype=np.float32)])
    v = normal(303, g.size)
    for sub in SUBOPS:
        run(gpu, sub, v, g)


def test_glu_rejections_leave_output_untouched(gpu):
    k = eh.Kernel()
    d_in = torch.ones(6, dtype=torch.float32, device=gpu)
    d_out = torch.full((3,), 9.0, dtype=torch.float32, device=gpu)
    cases = [
        (eh.OpGlu(d_in, d_out, eh.GluSubOp.SWIGLU, input_len=5, output_len=2), eh.Status.SHAPE_MISMATCH),
        (eh.OpGlu(d_in, d_out, eh.GluSubOp.SWIGLU, input_len=0, output_len=0), eh.Status.SHAPE_MISMATCH),
        (eh.OpGlu(d_in, d_out, eh.GluSubOp.SWIGLU, input_len=6, output_len=2), eh.Status.SHAPE_MISMATCH),
        (eh.OpGlu(d_in, d_out, 6), eh.Status.UNEXPECTED_EVENT),
        (eh.OpGlu(int(d_in.data_ptr()), d_out, eh.GluSubOp.SWIGLU, input_len=6), eh.Status.OK),
    ]
    for ev, want in cases[:4]:
        assert k.process_event(ev) == want
        assert torch.equal(d_out.cpu(), torch.full((3,), 9.0))
    # output overlapping the input is refused
    assert k.process_event(eh.OpGlu(d_in, d_in[3:], eh.GluSubOp.SWIGLU)) == eh.Status.INVALID_ARGUMENT
    assert k.process_event(cases[4][0]) == cases[4][1]
