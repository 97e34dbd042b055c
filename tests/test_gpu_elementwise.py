"""GPU parity: elementwise family vs the CPU oracle, bit-exact.

Covers binary add/sub/mul/div (binary.rs), row broadcast (broadcast.rs),
4-D modulo broadcast (OpRepeat + binary), unary silu/gelu/exp/tanh/elu/abs/
neg/relu (unary.rs), scale (activation.rs) and the fused SwiGLU, on the
BASELINE configs' shapes plus ragged sizes and strided / permuted /
implicit-stride / zero-stride layouts.  Every comparison is bit-exact
(any NaN matches any NaN).
"""
import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from helpers import Pair, assert_bits_equal, normal, row_major_nb, uniform

pytestmark = pytest.mark.gpu

BIN_EV = {orc.ADD: eh.OpAdd, orc.SUB: eh.OpSub, orc.MUL: eh.OpMul, orc.DIV: eh.OpDiv}


def edge_values():
    """Specials: signed zeros, infinities, NaN, denormals, extremes, and
    values around the formulas' branch points."""
    f = np.float32
    vals = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.1754942e-38, -1.1754942e-38, 3.4028235e38,
            -3.4028235e38, 1.0, -1.0, 10.0, -10.0, np.nextafter(f(10), f(0)), np.nextafter(f(-10), f(0)), 88.0,
            88.72283, 88.7229, -87.33654, -103.97208, -103.9721, -104.0, 0.5 * np.log(2), 1.5 * np.log(2), 22.0,
            -22.0, 2.0 ** -25, 2.0 ** -56, 0.25, 65504.0, 65520.0, -65520.0, 6.1e-5, 5.96e-8, 2.98e-8]
    return np.array(vals, dtype=np.float32)


def fp16_neighbourhood():
    """Every f16 value in (-10, 10) and the f32 midpoints between neighbours
    (the round-to-nearest-even ties GELU's input rounding must get right)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h) & (np.abs(h) < 10)]
    h = np.unique(h)
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    return np.concatenate([h, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])


def run_binary(gpu, op, a: Pair, b: Pair, o: Pair, ev=None):
    for p in (a, b, o):
        p.to(gpu)
    k = eh.Kernel()
    ev = ev or BIN_EV[op]
    st = k.process_event(ev(a.pview(), b.pview(), o.pview(mut=True)))
    assert st == eh.Status.OK, eh.last_error()
    want = o.host.copy()
    ov = orc.view(want, o.ne, o.nb)
    assert orc.binary(op, a.oview(), b.oview(), ov) == orc.OK
    assert_bits_equal(o.result(), want, f"binary op {op}")


# add, sub and mul stream 512 float4 per wave, 2048 per workgroup: 2049, 8191, 8196 and 24579
# end inside a wave's and a workgroup's span
@pytest.mark.parametrize("op", [orc.ADD, orc.SUB, orc.MUL, orc.DIV])
@pytest.mark.parametrize("n", [1, 3, 4, 5, 255, 1023, 4097, 11008 * 512, 2049, 8191, 8196, 24579])
def test_binary_dense(gpu, op, n):
    a = Pair(uniform(11 + n, n), [n, 1, 1, 1])
    b = Pair(uniform(17 + n, n), [n, 1, 1, 1])
    o = Pair(np.zeros(n, np.float32), [n, 1, 1, 1])
    run_binary(gpu, op, a, b, o)


@pytest.mark.parametrize("op", [orc.ADD, orc.MUL, orc.DIV])
def test_binary_edge_values(gpu, op):
    e = edge_values()
    a_vals = np.repeat(e, e.size)
    b_vals = np.tile(e, e.size)
    n = a_vals.size
    run_binary(gpu, op, Pair(a_vals, [n, 1, 1, 1]), Pair(b_vals, [n, 1, 1, 1]), Pair(np.zeros(n, np.float32), [n, 1, 1, 1]))


def test_binary_layouts(gpu):
    # strided (every other element), reshaped equal-count, implicit nb[0]==0,
    # and an explicit zero stride on a singleton dim (binary contract only)
    n0, n1 = 37, 9
    sparse = Pair(uniform(1, 2 * n0 * n1), [n0, n1, 1, 1], [8, 8 * n0, 8 * n0 * n1, 8 * n0 * n1])
    dense = Pair(uniform(2, n0 * n1), [n0, n1, 1, 1])
    reshaped = Pair(uniform(3, n0 * n1), [n1, n0, 1, 1])
    out = Pair(np.zeros(n0 * n1, np.float32), [n0 * n1, 1, 1, 1])
    run_binary(gpu, orc.ADD, sparse, reshaped, out)
    implicit = Pair(uniform(4, n0 * n1), [n0, n1, 1, 1], [0, 0, 0, 0])
    run_binary(gpu, orc.MUL, implicit, dense, Pair(np.zeros(n0 * n1, np.float32), [n0, n1, 1, 1], [0, 0, 0, 0]))
    zs = Pair(uniform(5, n0 * n1), [n0, n1, 1, 1], [4, 4 * n0, 0, 0])
    run_binary(gpu, orc.SUB, zs, dense, Pair(np.zeros(n0 * n1, np.float32), [n0, n1, 1, 1]))
    # transposed (permuted) operand against dense output
    t = Pair(uniform(6, n0 * n1), [n1, n0, 1, 1]).host
    tp = Pair(t, [n0, n1, 1, 1], [4 * n1, 4, 4 * n0 * n1, 4 * n0 * n1])
    run_binary(gpu, orc.DIV, tp, dense, Pair(np.zeros(n0 * n1, np.float32), [n0, n1, 1, 1]))


def test_binary_in_place(gpu):
    n = 100003
    a = Pair(uniform(7, n), [n, 1, 1, 1]).to(gpu)
    b = Pair(uniform(8, n), [n, 1, 1, 1]).to(gpu)
    want = a.host.copy()
    assert orc.binary(orc.ADD, orc.view(want, a.ne), b.oview(), orc.view(want, a.ne)) == orc.OK
    st = eh.Kernel().process_event(eh.OpAdd(a.pview(), b.pview(), a.pview(mut=True)))
    assert st == eh.Status.OK
    assert_bits_equal(a.result(), want, "in-place add")


@pytest.mark.parametrize("op", [orc.ADD, orc.MUL])
@pytest.mark.parametrize("ne0,rows", [(4096, 512), (3, 2), (1001, 7), (4, 1000), (8192, 3)])
def test_broadcast_row(gpu, op, ne0, rows):
    a = Pair(uniform(21, ne0 * rows), [ne0, rows, 1, 1]).to(gpu)
    b = Pair(uniform(22, ne0), [ne0, 1, 1, 1]).to(gpu)
    o = Pair(np.zeros(ne0 * rows, np.float32), [ne0, rows, 1, 1]).to(gpu)
    ev = eh.OpAddBroadcastRow if op == orc.ADD else eh.OpMulBroadcastRow
    st = eh.Kernel().process_event(ev(a.pview(), b.pview(), o.pview(mut=True)))
    assert st == eh.Status.OK, eh.last_error()
    want = o.host.copy()
    assert orc.broadcast_row(op, a.oview(), b.oview(), orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, "broadcast_row")


def test_broadcast_row_config1_equals_4d_broadcast(gpu):
    # special case: 4-D broadcast with src1 = [ne0,1,1,1] must equal OpAddBroadcastRow
    ne0, rows = 4096, 512
    a = Pair(uniform(31, ne0 * rows), [ne0, rows, 1, 1]).to(gpu)
    b = Pair(uniform(32, ne0), [ne0, 1, 1, 1]).to(gpu)
    o1 = Pair(np.zeros(ne0 * rows, np.float32), [ne0, rows, 1, 1]).to(gpu)
    o2 = Pair(np.zeros(ne0 * rows, np.float32), [ne0, rows, 1, 1]).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpAddBroadcastRow(a.pview(), b.pview(), o1.pview(mut=True))) == eh.Status.OK
    assert k.process_event(eh.OpBinaryBroadcast(eh.BinaryOp.ADD, a.pview(), b.pview(), o2.pview(mut=True))) == eh.Status.OK
    assert_bits_equal(o1.result(), o2.result(), "row broadcast vs 4-D broadcast")


BCAST_CASES = [
    # (src0 storage ne, permutation axes for the view, src1 ne)
    ([128, 32, 64, 8], [0, 2, 1, 3], [128, 1, 32, 1]),  # config 5b: dims 1<->2 swapped
    ([64, 16, 8, 4], None, [64, 16, 8, 4]),             # equal shapes == OpMul
    ([64, 16, 8, 4], None, [1, 16, 1, 4]),              # dim-0 splat
    ([60, 6, 10, 3], None, [60, 3, 5, 1]),              # modulo repeat (divisors)
    ([33, 5, 7, 2], [0, 2, 1, 3], [33, 1, 5, 2]),       # ragged ne0 -> general path
    ([16, 8, 4, 2], [1, 0, 2, 3], [1, 16, 1, 1]),       # non-contiguous dim 0
]


@pytest.mark.parametrize("op", [orc.MUL, orc.ADD, orc.SUB, orc.DIV])
@pytest.mark.parametrize("case", BCAST_CASES, ids=lambda c: "x".join(map(str, c[0])))
def test_binary_broadcast_4d(gpu, op, case):
    sne, axes, b_ne = case
    n = int(np.prod(sne))
    storage = normal(41, n)
    nb = row_major_nb(sne)
    if axes is not None:
        ne = [sne[a] for a in axes]
        nb = [nb[a] for a in axes]
    else:
        ne = list(sne)
    a = Pair(storage, ne, nb).to(gpu)
    b = Pair(uniform(42, int(np.prod(b_ne)), 0.5, 1.5), b_ne).to(gpu)
    o = Pair(np.zeros(n, np.float32), ne).to(gpu)
    st = eh.Kernel().process_event(eh.OpBinaryBroadcast(eh.BinaryOp(op), a.pview(), b.pview(), o.pview(mut=True)))
    assert st == eh.Status.OK, eh.last_error()
    want = o.host.copy()
    assert orc.binary_bcast(op, a.oview(), b.oview(), orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, f"4-D broadcast {case}")


UNARY = {"abs": 0, "neg": 2, "tanh": 4, "elu": 5, "relu": 6, "gelu": 8, "silu": 10, "exp": 13}


@pytest.mark.parametrize("name", list(UNARY))
def test_unary_config2_and_edges(gpu, name):
    x = np.concatenate([normal(51, 11008 * 512), edge_values(), normal(52, 4099, 30.0)])
    n = x.size
    a = Pair(x, [n, 1, 1, 1]).to(gpu)
    o = Pair(np.zeros(n, np.float32), [n, 1, 1, 1]).to(gpu)
    st = eh.Kernel().process_event(eh.OpUnary(eh.UnarySubOp(UNARY[name]), a.pview(), o.pview(mut=True)))
    assert st == eh.Status.OK, eh.last_error()
    want = np.zeros(n, np.float32)
    assert orc.unary(UNARY[name], a.oview(), orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, name)


@pytest.mark.parametrize("name", ["gelu", "silu", "exp", "tanh"])
def test_unary_fp16_grid(gpu, name):
    x = fp16_neighbourhood()
    n = x.size
    a = Pair(x, [n, 1, 1, 1]).to(gpu)
    o = Pair(np.zeros(n, np.float32), [n, 1, 1, 1]).to(gpu)
    assert eh.Kernel().process_event(eh.OpUnary(eh.UnarySubOp(UNARY[name]), a.pview(), o.pview(mut=True))) == eh.Status.OK
    want = np.zeros(n, np.float32)
    assert orc.unary(UNARY[name], a.oview(), orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, name)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 255, 1023, 1025, 262147, 2 * 2048 * 256 * 4 + 7])
def test_heavy_unary_ragged_sizes(gpu, n):
    """The libm-based unary formulas walk a resident grid (one float4 per
    thread per step, a scalar tail): sizes below one float4, one short of and
    past a workgroup, and past one resident generation of 2048 x 256 threads."""
    x = normal(53 + n % 17, n, 8.0)
    a = Pair(x, [n, 1, 1, 1]).to(gpu)
    for name in ("silu", "exp", "tanh", "elu"):
        o = Pair(np.zeros(n, np.float32), [n, 1, 1, 1]).to(gpu)
        st = eh.Kernel().process_event(eh.OpUnary(eh.UnarySubOp(UNARY[name]), a.pview(), o.pview(mut=True)))
        assert st == eh.Status.OK, eh.last_error()
        want = np.zeros(n, np.float32)
        assert orc.unary(UNARY[name], a.oview(), orc.view(want, o.ne)) == orc.OK
        assert_bits_equal(o.result(), want, f"{name} n={n}")


def test_exp_dense_sweep(gpu):
    # every 97th f32 bit pattern: ~44M inputs across the whole float line
    u = np.arange(0, 2 ** 32, 97, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    n = x.size
    a = Pair(x, [n, 1, 1, 1]).to(gpu)
    o = Pair(np.zeros(n, np.float32), [n, 1, 1, 1]).to(gpu)
    for name in ("exp", "silu", "tanh"):
        assert eh.Kernel().process_event(eh.OpUnary(eh.UnarySubOp(UNARY[name]), a.pview(), o.pview(mut=True))) == eh.Status.OK
        want = np.zeros(n, np.float32)
        assert orc.unary(UNARY[name], a.oview(), orc.view(want, o.ne)) == orc.OK
        assert_bits_equal(o.result(), want, name)


@pytest.mark.parametrize("which", ["silu", "gelu"])
def test_dedicated_events_strided(gpu, which):
    n0, n1 = 129, 33
    a = Pair(normal(61, 3 * n0 * n1, 3.0), [n0, n1, 1, 1], [12, 12 * n0, 12 * n0 * n1, 12 * n0 * n1]).to(gpu)
    o = Pair(np.zeros(n0 * n1, np.float32), [n1, n0, 1, 1]).to(gpu)  # equal count, other shape
    ev = eh.OpSilu if which == "silu" else eh.OpGelu
    assert eh.Kernel().process_event(ev(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = np.zeros(n0 * n1, np.float32)
    assert orc.unary_event(10 if which == "silu" else 8, a.oview(), orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, which)


def test_swiglu_config2(gpu):
    n = 11008 * 512
    gate = Pair(normal(71, n), [11008, 512, 1, 1]).to(gpu)
    up = Pair(normal(72, n), [11008, 512, 1, 1]).to(gpu)
    out = Pair(np.zeros(n, np.float32), [11008, 512, 1, 1]).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpSwiglu(gate.pview(), up.pview(), out.pview(mut=True))) == eh.Status.OK
    want = np.zeros(n, np.float32)
    assert orc.swiglu(gate.oview(), up.oview(), orc.view(want, out.ne)) == orc.OK
    assert_bits_equal(out.result(), want, "swiglu")
    # the unfused chain (OpSilu then OpMul) gives the same bits
    tmp = Pair(np.zeros(n, np.float32), out.ne).to(gpu)
    out2 = Pair(np.zeros(n, np.float32), out.ne).to(gpu)
    assert k.process_event(eh.OpSilu(gate.pview(), tmp.pview(mut=True))) == eh.Status.OK
    assert k.process_event(eh.OpMul(tmp.pview(), up.pview(), out2.pview(mut=True))) == eh.Status.OK
    assert_bits_equal(out2.result(), want, "silu then mul")


def test_scale(gpu):
    n = 1 << 20
    x = np.concatenate([normal(81, n), edge_values()])
    a = Pair(x, [x.size, 1, 1, 1]).to(gpu)
    o = Pair(np.zeros(x.size, np.float32), a.ne).to(gpu)
    s = float(np.float32(1.0 / np.sqrt(128.0)))
    assert eh.Kernel().process_event(eh.OpScale(a.pview(), o.pview(mut=True), s)) == eh.Status.OK
    want = np.zeros(x.size, np.float32)
    assert orc.scale(a.oview(), orc.view(want, a.ne), s) == orc.OK
    assert_bits_equal(o.result(), want, "scale")
