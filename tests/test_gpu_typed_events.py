"""GPU parity: the typed events of activation.rs (OpClamp, OpLeakyRelu,
OpSiluBack), elementwise.rs (OpAdd1, OpAcc), diag.rs (OpDiag,
OpDiagMaskInf, OpDiagMaskZero) and group_norm.rs (OpGroupNorm, OpL2Norm)
through the C ABI against the oracle: bit-exact except group_norm (f64 sums
as a tree: 1e-5 relative, as rms_norm)."""
import numpy as np
import pytest
import torch

import emel_hip as eh
import oracle as orc
from helpers import Pair, assert_bits_equal, assert_close_rel

pytestmark = pytest.mark.gpu


def values(seed, n):
    g = np.random.Generator(np.random.PCG64(seed))
    x = (g.standard_normal(n) * 4).astype(np.float32)
    special = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, 1e-40, -3e38, 3e38], np.float32)
    x[:min(n, 8)] = special[:min(n, 8)]
    return x


@pytest.mark.parametrize("layout", ["dense", "strided"])
def test_activation_events(gpu, layout):
    n = 4096
    x = values(601, 2 * n)
    ne, nb = ([64, 64, 1, 1], None) if layout == "dense" else ([64, 64, 1, 1], [8, 512, 32768, 32768])
    k = eh.Kernel()
    for lo, hi in ((-1.0, 1.0), (2.0, -2.0)):  # min > max too
        a = Pair(x, ne, nb).to(gpu)
        o = Pair(np.zeros(n, np.float32), [64, 64, 1, 1]).to(gpu)
        assert k.process_event(eh.OpClamp(a.pview(), o.pview(mut=True), lo, hi)) == eh.Status.OK, eh.last_error()
        want = np.zeros(n, np.float32)
        assert orc.clamp(a.oview(), orc.view(want, o.ne), lo, hi) == orc.OK
        assert_bits_equal(o.result(), want, f"clamp {lo} {hi}")
    a = Pair(x, ne, nb).to(gpu)
    o = Pair(np.zeros(n, np.float32), [64, 64, 1, 1]).to(gpu)
    assert k.process_event(eh.OpLeakyRelu(a.pview(), o.pview(mut=True), 0.01)) == eh.Status.OK
    want = np.zeros(n, np.float32)
    assert orc.leaky_relu(a.oview(), orc.view(want, o.ne), 0.01) == orc.OK
    assert_bits_equal(o.result(), want, "leaky_relu")
    gr = Pair(values(602, 2 * n), ne, nb).to(gpu)
    assert k.process_event(eh.OpSiluBack(a.pview(), gr.pview(), o.pview(mut=True))) == eh.Status.OK
    assert orc.silu_back(a.oview(), gr.oview(), orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, "silu_back")
    assert k.process_event(eh.OpAdd1(a.pview(), -0.75, o.pview(mut=True))) == eh.Status.OK
    assert orc.add1(a.oview(), -0.75, orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, "add1")


def test_activation_guards(gpu):
    a = Pair(np.ones(8, np.float32), [8, 1, 1, 1]).to(gpu)
    o = Pair(np.full(8, 9.0, np.float32), [4, 2, 1, 1]).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpClamp(a.pview(), o.pview(mut=True), 0.0, 1.0)) == eh.Status.SHAPE_MISMATCH
    assert k.process_event(eh.OpSiluBack(a.pview(), a.pview(), o.pview(mut=True))) == eh.Status.SHAPE_MISMATCH
    assert k.process_event(eh.OpAdd1(a.pview(), 1.0, o.pview(mut=True))) == eh.Status.SHAPE_MISMATCH
    assert (o.result() == 9.0).all()


@pytest.mark.parametrize("n,nu,offset", [(6, 2, 2), (100003, 4099, 50000), (4096, 4096, 0), (7, 1, 6)])
def test_acc(gpu, n, nu, offset):
    base = values(611, n)
    upd = values(612, nu)
    b = Pair(base, [n, 1, 1, 1]).to(gpu)
    k = eh.Kernel()
    o = Pair(np.zeros(n, np.float32), [n, 1, 1, 1]).to(gpu)
    u = Pair(upd, [nu, 1, 1, 1]).to(gpu)
    assert k.process_event(eh.OpAcc(b.pview(), u.pview(), o.pview(mut=True), offset)) == eh.Status.OK, eh.last_error()
    want = np.zeros(n, np.float32)
    assert orc.acc(b.oview(), u.oview(), orc.view(want, o.ne), offset) == orc.OK
    assert_bits_equal(o.result(), want, "acc")
    # in place on the base
    assert k.process_event(eh.OpAcc(b.pview(), u.pview(), b.pview(mut=True), offset)) == eh.Status.OK
    assert_bits_equal(b.result(), want, "acc in place")


def test_acc_guards(gpu):
    b = Pair(np.ones(4, np.float32), [4, 1, 1, 1]).to(gpu)
    u = Pair(np.ones(2, np.float32), [2, 1, 1, 1]).to(gpu)
    o = Pair(np.full(4, 9.0, np.float32), [4, 1, 1, 1]).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpAcc(b.pview(), u.pview(), o.pview(mut=True), 3)) == eh.Status.INVALID_OFFSET
    s = Pair(np.ones(8, np.float32), [4, 1, 1, 1], [8, 32, 32, 32]).to(gpu)
    assert k.process_event(eh.OpAcc(s.pview(), u.pview(), o.pview(mut=True), 0)) == eh.Status.INVALID_VIEW
    o3 = Pair(np.full(3, 9.0, np.float32), [3, 1, 1, 1]).to(gpu)
    assert k.process_event(eh.OpAcc(b.pview(), u.pview(), o3.pview(mut=True), 0)) == eh.Status.SHAPE_MISMATCH
    assert (o.result() == 9.0).all() and (o3.result() == 9.0).all()


@pytest.mark.parametrize("n", [1, 2, 37, 512])
def test_diag_family(gpu, n):
    k = eh.Kernel()
    x = values(621, n)
    xt = torch.from_numpy(x).to(gpu)
    ot = torch.full((n * n,), 9.0, device=gpu)
    assert k.process_event(eh.OpDiag(xt, ot)) == eh.Status.OK, eh.last_error()
    want = np.zeros(n * n, np.float32)
    assert orc.diag(x, want) == orc.OK
    assert_bits_equal(ot.cpu().numpy(), want, "diag")
    sq = values(622, n * n)
    for inf, cls in ((True, eh.OpDiagMaskInf), (False, eh.OpDiagMaskZero)):
        for past in (0, 3, n + 5):
            st = torch.from_numpy(sq).to(gpu)
            mt = torch.zeros(n * n, device=gpu)
            assert k.process_event(cls(st, mt, past)) == eh.Status.OK
            want = np.zeros(n * n, np.float32)
            assert orc.diag_mask(inf, sq, want, past) == orc.OK
            assert_bits_equal(mt.cpu().numpy(), want, f"diag_mask inf={inf} past={past}")
            assert k.process_event(cls(st, st, past)) == eh.Status.OK  # in place
            assert_bits_equal(st.cpu().numpy(), want, "diag_mask in place")


def test_diag_guards(gpu):
    k = eh.Kernel()
    x = torch.ones(2, device=gpu)
    bad = torch.full((3,), 7.0, device=gpu)
    assert k.process_event(eh.OpDiag(x, bad)) == eh.Status.INVALID_SHAPE
    sq = torch.ones(4, device=gpu)
    keep = torch.full((4,), 8.0, device=gpu)
    assert k.process_event(eh.OpDiagMaskZero(sq, keep, -1)) == eh.Status.INVALID_SHAPE
    assert k.process_event(eh.OpDiagMaskInf(sq, torch.zeros(5, device=gpu), 0)) == eh.Status.INVALID_SHAPE
    assert (bad.cpu() == 7).all() and (keep.cpu() == 8).all()


@pytest.mark.parametrize("W,H,C,B,G", [(2, 1, 4, 1, 2), (64, 64, 32, 2, 8), (7, 5, 12, 3, 4), (256, 256, 16, 1, 1)])
def test_group_norm(gpu, W, H, C, B, G):
    g = np.random.Generator(np.random.PCG64(631 + W))
    x = (g.standard_normal(W * H * C * B) * 3 + 0.5).astype(np.float32)
    ne = [W, H, C, B]
    a = Pair(x, ne).to(gpu)
    o = Pair(np.zeros_like(x), ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpGroupNorm(a.pview(), o.pview(mut=True), G, 1e-5)) == eh.Status.OK, \
        eh.last_error()
    want = np.zeros_like(x)
    assert orc.group_norm(a.oview(), orc.view(want, ne), G, 1e-5) == orc.OK
    assert_close_rel(o.result(), want, 1e-5, "group_norm", atol=1e-6)


def test_group_norm_strided_and_guards(gpu):
    g = np.random.Generator(np.random.PCG64(641))
    W, H, C, B = 6, 4, 8, 2
    x = g.standard_normal(2 * W * H * C * B).astype(np.float32)
    nb = [8, 8 * W, 8 * W * H, 8 * W * H * C]
    a = Pair(x, [W, H, C, B], nb).to(gpu)
    o = Pair(np.zeros(W * H * C * B, np.float32), [W, H, C, B]).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpGroupNorm(a.pview(), o.pview(mut=True), 4, 0.01)) == eh.Status.OK, eh.last_error()
    want = np.zeros(W * H * C * B, np.float32)
    assert orc.group_norm(a.oview(), orc.view(want, o.ne), 4, 0.01) == orc.OK
    assert_close_rel(o.result(), want, 1e-5, "strided group_norm", atol=1e-6)
    keep = Pair(np.full(W * H * C * B, 7.0, np.float32), [W, H, C, B]).to(gpu)
    assert k.process_event(eh.OpGroupNorm(a.pview(), keep.pview(mut=True), 3, 0.0)) == eh.Status.INVALID_PARAMETERS
    assert k.process_event(eh.OpGroupNorm(a.pview(), keep.pview(mut=True), 2, -1.0)) == eh.Status.INVALID_PARAMETERS
    assert (keep.result() == 7.0).all()


def test_l2_norm(gpu):
    k = eh.Kernel()
    for n, seed in ((3, None), (1000, 651), (65536, 652)):
        x = np.array([3.0, 4.0, 0.0], np.float32) if seed is None else \
            np.random.Generator(np.random.PCG64(seed)).standard_normal(n).astype(np.float32)
        a = Pair(x, [n, 1, 1, 1]).to(gpu)
        o = Pair(np.zeros(n, np.float32), [n, 1, 1, 1]).to(gpu)
        assert k.process_event(eh.OpL2Norm(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
        want = np.zeros(n, np.float32)
        assert orc.l2_norm(a.oview(), orc.view(want, o.ne)) == orc.OK
        assert_bits_equal(o.result(), want, f"l2_norm {n}")
    z = Pair(np.zeros(4, np.float32), [4, 1, 1, 1]).to(gpu)
    keep = Pair(np.full(4, 5.0, np.float32), [4, 1, 1, 1]).to(gpu)
    assert k.process_event(eh.OpL2Norm(z.pview(), keep.pview(mut=True))) == eh.Status.ZERO_NORM
    assert (keep.result() == 5.0).all()
