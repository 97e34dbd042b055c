"""GPU parity: sum_rows, per-row argmax and whole-tensor sum / mean / argmax.

argmax indices are compared exactly (ties and NaNs included); sums within
BASELINE's 1e-5 relative tolerance (f64 accumulation in a different order),
with an absolute floor of 1e-12 * sum|x| for rows whose sum nearly cancels.
"""
import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from helpers import Pair, assert_close_rel, normal

pytestmark = pytest.mark.gpu


def planted_logits(cols, rows, seed):
    """N(0,1) rows with a planted maximum at a seeded index and, in every
    other row, a tie at a higher index (the lower index must win)."""
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal(cols * rows, dtype=np.float64).astype(np.float32).reshape(rows, cols)
    where = g.integers(0, cols, rows)
    for r in range(rows):
        x[r, where[r]] = np.float32(8.0 + r * 1e-3)
        if r % 2 == 0 and where[r] + 1 < cols:
            tie = g.integers(where[r] + 1, cols)
            x[r, tie] = x[r, where[r]]
    return x.reshape(-1), where


def run_argmax_rows(gpu, x, ne, nb=None):
    a = Pair(x, ne, nb).to(gpu)
    rows = int(np.prod(ne[1:]))
    o = Pair(np.full(rows, -7, np.int32), [1, ne[1], ne[2], ne[3]]).to(gpu)
    assert eh.Kernel().process_event(eh.OpArgmaxRows(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = np.full(rows, -7, np.int32)
    assert orc.argmax_rows(a.oview(), orc.view(want, o.ne)) == orc.OK
    got = o.result()
    assert (got == want).all(), (np.flatnonzero(got != want)[:5], got[got != want][:5], want[got != want][:5])
    return got


def test_argmax_rows_config5(gpu):
    cols, rows = 151936, 64
    x, where = planted_logits(cols, rows, 201)
    got = run_argmax_rows(gpu, x, [cols, rows, 1, 1])
    assert (got == where).all()


@pytest.mark.parametrize("cols,rows", [(1, 3), (5, 2), (1024, 1), (4095, 3), (100003, 2), (4096, 4096)])
def test_argmax_rows_sizes(gpu, cols, rows):
    x, _ = planted_logits(cols, rows, 202 + cols)
    run_argmax_rows(gpu, x, [cols, rows, 1, 1])


def test_argmax_rows_nan_inf_ties(gpu):
    cols = 50000
    rows = []
    base = np.zeros(cols, np.float32)
    r = base.copy(); r[0] = np.nan; r[10] = 5.0; rows.append(r)                 # NaN at column 0 -> 0
    r = base.copy(); r[3] = np.nan; r[40000] = 1.0; rows.append(r)              # later NaN is skipped
    r = np.full(cols, -np.inf, np.float32); rows.append(r)                     # all -inf -> 0
    r = np.full(cols, -np.inf, np.float32); r[7] = np.nan; r[49999] = -1.0; rows.append(r)
    r = base.copy(); r[5] = -0.0; r[2] = 0.0; rows.append(r)                   # +-0 tie -> lowest index
    r = base.copy(); r[123] = np.inf; r[45000] = np.inf; rows.append(r)
    r = np.full(cols, np.nan, np.float32); rows.append(r)
    r = np.full(cols, 3.0, np.float32); rows.append(r)                          # all equal -> 0
    x = np.concatenate(rows)
    got = run_argmax_rows(gpu, x, [cols, len(rows), 1, 1])
    assert list(got) == [0, 40000, 0, 49999, 0, 123, 0, 0]


def test_argmax_column0_nan_in_split_rows(gpu):
    # rows long enough to be split across workgroups: a NaN in column 0 must
    # decide the row even against a later +inf in another chunk
    cols, rows = 151936, 4
    x, where = planted_logits(cols, rows, 271)
    x = x.reshape(rows, cols)
    x[0, 0] = np.nan; x[0, 70000] = np.inf      # -> 0
    x[1, 0] = np.nan                             # -> 0
    x[2, 1] = np.nan; x[2, 100000] = np.inf     # -> 100000
    x[3, 0] = -np.inf                            # -> the planted maximum
    got = run_argmax_rows(gpu, x.reshape(-1), [cols, rows, 1, 1])
    assert list(got) == [0, 0, 100000, where[3]]
    # the whole-tensor argmax, dense and through the ordinal decode (a
    # transposed view whose ordinal 0 is still x[0, 0])
    for ne, nb in (([cols * rows, 1, 1, 1], None), ([rows, cols, 1, 1], [4 * cols, 4, 4 * cols * rows, 4 * cols * rows])):
        a = Pair(x.reshape(-1), ne, nb).to(gpu)
        o = Pair(np.full(1, -7, np.float32), [1, 1, 1, 1]).to(gpu)
        assert eh.Kernel().process_event(eh.OpArgmax(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
        want = np.full(1, -7, np.float32)
        assert orc.argmax(a.oview(), orc.view(want, [1, 1, 1, 1])) == orc.OK
        assert want[0] == 0.0 and o.result()[0] == want[0], (o.result(), want)


def test_argmax_rows_strided(gpu):
    cols, rows, pad = 999, 6, 1024
    x = normal(211, pad * rows * 2)
    run_argmax_rows(gpu, x, [cols, rows, 1, 1], [8, 8 * pad, 8 * pad * rows, 8 * pad * rows])


def sum_rows_check(gpu, x, ne, nb=None):
    a = Pair(x, ne, nb).to(gpu)
    o = Pair(np.zeros(int(np.prod(ne[1:])), np.float32), [1, ne[1], ne[2], ne[3]]).to(gpu)
    assert eh.Kernel().process_event(eh.OpSumRows(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = np.zeros(o.host.size, np.float32)
    assert orc.sum_rows(a.oview(), orc.view(want, o.ne)) == orc.OK
    got = o.result().astype(np.float64)
    # condition-number floor: the f64 sums can differ by ~1e-16 * sum|x|
    absx = np.abs(x.astype(np.float64))
    floor = 1e-12 * max(absx.sum(), 1.0)
    ok = np.abs(got - want) <= 1e-5 * np.abs(want) + floor
    assert ok.all(), (got[~ok][:4], want[~ok][:4])


def test_sum_rows_config5(gpu):
    x, _ = planted_logits(151936, 64, 221)
    sum_rows_check(gpu, x, [151936, 64, 1, 1])


@pytest.mark.parametrize("ne", [[3, 2, 1, 1], [1, 7, 1, 1], [4096, 16, 2, 2], [10001, 3, 1, 2]])
def test_sum_rows_shapes(gpu, ne):
    sum_rows_check(gpu, normal(231, int(np.prod(ne))), ne)


def test_sum_rows_strided(gpu):
    cols, rows = 777, 13
    sum_rows_check(gpu, normal(241, 3 * cols * rows), [cols, rows, 1, 1], [12, 12 * cols, 12 * cols * rows, 12 * cols * rows])


@pytest.mark.parametrize("ne,nb", [([151936, 64, 1, 1], None), ([3, 2, 1, 1], None), ([17, 5, 3, 1], [0, 0, 0, 0]),
                                   ([9, 4, 2, 1], [8, 72, 288, 576])])
def test_scalar_reductions(gpu, ne, nb):
    n = int(np.prod(ne))
    span = n if nb is None or nb[0] == 0 else (sum((ne[d] - 1) * nb[d] for d in range(4)) // 4 + 1)
    x, _ = planted_logits(span, 1, 251)
    a = Pair(x, ne, nb).to(gpu)
    k = eh.Kernel()
    for ev, fn, exact in ((eh.OpArgmax, orc.argmax, True), (eh.OpSum, orc.sum_, False), (eh.OpMean, orc.mean, False)):
        o = Pair(np.zeros(1, np.float32), [1, 1, 1, 1]).to(gpu)
        assert k.process_event(ev(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
        want = np.zeros(1, np.float32)
        assert fn(a.oview(), orc.view(want, [1, 1, 1, 1])) == orc.OK
        got = o.result()
        if exact:
            assert got[0] == want[0], (got, want)
        else:
            floor = 1e-12 * np.abs(x.astype(np.float64)).sum()
            assert abs(float(got[0]) - float(want[0])) <= 1e-5 * abs(float(want[0])) + floor, (got, want)


def _alternating_launches(gpu, event, oracle_fn, cols, rows, out_dtype, seeds, launches=12):
    """Back-to-back launches, no synchronisation between them, alternating
    between inputs that differ in every row, each into its own output.  A
    merge that read a partial left by the previous launch (same slots, other
    data) would give that launch's row result, so every output is checked
    against the oracle."""
    import torch

    ins = []
    for sd in seeds:
        x, _ = planted_logits(cols, rows, sd)
        ins.append(Pair(x, [cols, rows, 1, 1]).to(gpu))
    outs = [Pair(np.zeros(rows, out_dtype), [1, rows, 1, 1]).to(gpu) for _ in range(launches)]
    k = eh.Kernel(synchronous=False)
    for i in range(launches):
        assert k.process_event(event(ins[i % len(ins)].pview(), outs[i].pview(mut=True))) == eh.Status.OK
    torch.cuda.synchronize()
    wants = []
    for a in ins:
        w = np.zeros(rows, out_dtype)
        assert oracle_fn(a.oview(), orc.view(w, [1, rows, 1, 1])) == orc.OK
        wants.append(w)
    for i in range(launches):
        got, want = outs[i].result(), wants[i % len(ins)]
        if out_dtype == np.int32:
            assert (got == want).all(), (i, np.flatnonzero(got != want)[:5])
        else:
            assert_close_rel(got, want, 1e-5, f"launch {i}", atol=1e-12 * 4 * cols)
    return wants


@pytest.mark.parametrize("cols,rows", [(151936, 64),   # config 5: 32 chunks per row, one merge level
                                       (600000, 4)])   # 512 chunks per row: two merge levels
def test_alternating_inputs_argmax_rows(gpu, cols, rows):
    wants = _alternating_launches(gpu, eh.OpArgmaxRows, orc.argmax_rows, cols, rows, np.int32, (261, 262))
    assert (wants[0] != wants[1]).all()  # every row's answer differs between the two inputs


@pytest.mark.parametrize("cols,rows", [(151936, 64), (600000, 4)])
def test_alternating_inputs_sum_rows(gpu, cols, rows):
    wants = _alternating_launches(gpu, eh.OpSumRows, orc.sum_rows, cols, rows, np.float32, (263, 264))
    assert (wants[0] != wants[1]).all()


def _f32_bits(u):
    return np.array(u, np.uint32).view(np.float32)


@pytest.mark.parametrize("cols,rows", [(151936, 12),   # 149 chunks of 1024 columns: one batch each
                                       (8192, 2048),   # one chunk per row, 2 batches (the second partial)
                                       (13004, 2100),  # 3 batches, the last partial
                                       (5124, 2048)])  # 2 batches, the last holding one float4
def test_argmax_rows_vector_path_corners(gpu, cols, rows):
    """The vector path's maximum tree, its search and the clamped last batch:
    maxima in an earlier batch tied by a later one, maxima in a chunk's last
    float4 (re-read by the lanes past the end), signalling NaNs, +-0 ties,
    rows that are all negative, all -inf or -inf with NaNs."""
    g = np.random.Generator(np.random.PCG64(281 + cols))
    x = g.standard_normal(cols * rows).astype(np.float32).reshape(rows, cols)
    snan_p, snan_n = _f32_bits(0x7F800001), _f32_bits(0xFFA00000)
    n = 0
    def row():
        nonlocal n
        n += 1
        return x[n - 1]
    r = row(); r[5] = 9.0; r[cols - 1] = 9.0                          # tie: first batch vs last float4 -> 5
    r = row(); r[cols - 1] = 9.0                                       # maximum in the chunk's last column
    r = row(); r[cols - 4] = 9.0                                       # ... its last float4's first column
    r = row(); r[1::7] = snan_p; r[100] = 20.0                         # signalling NaNs everywhere -> 100
    r = row(); r[:] = snan_n; r[0] = -5.0; r[cols // 2] = -1.0         # all sNaN but two values
    r = row(); r[:] = -np.abs(r) - 1.0; r[cols - 2] = -0.5             # all negative: no zero from a pad
    r = row(); r[:] = -1.0; r[3] = -0.0; r[cols - 1] = 0.0; r[cols // 2] = -0.0   # +-0 tie -> 3
    r = row(); r[:] = -np.inf                                          # all -inf -> 0
    r = row(); r[:] = np.nan; r[1] = -np.inf; r[cols - 3] = -np.inf    # NaN at 0 -> 0
    r = row(); r[:] = np.nan; r[0] = -np.inf; r[cols - 3] = -np.inf    # -> 0
    r = row(); r[:] = _f32_bits(0x7FC00001); r[0] = -2.0; r[cols - 1] = 1.0   # quiet NaNs -> cols-1
    r = row(); r[1280 * 4 + 1] = 50.0; r[2 * 1280 * 4 + 7 if 2 * 1280 * 4 + 7 < cols else 0] = 50.0
    got = run_argmax_rows(gpu, x.reshape(-1), [cols, rows, 1, 1])
    assert list(got[[0, 1, 2, 3, 6, 7, 8, 9, 10]]) == [5, cols - 1, cols - 4, 100, 3, 0, 0, 0, cols - 1], got[:12]


def test_sum_rows_non_finite(gpu):
    # f64 accumulation: NaN anywhere -> NaN; +inf and -inf -> NaN; one sign of
    # inf -> inf; finite values whose f64 sum exceeds the f32 range -> inf
    # when rounded; the order of the f64 tree cannot change these.
    for cols in (151936, 4096, 37):
        g = np.random.Generator(np.random.PCG64(431 + cols))
        rows = []
        def base():
            return g.standard_normal(cols).astype(np.float32)
        r = base(); r[0] = np.nan; rows.append(r)
        r = base(); r[cols // 2] = np.nan; r[1] = np.inf; rows.append(r)
        r = base(); r[cols // 3] = np.inf; rows.append(r)
        r = base(); r[cols // 3] = np.inf; r[-1] = -np.inf; rows.append(r)
        r = base(); r[-1] = -np.inf; rows.append(r)
        rows.append(np.full(cols, np.float32(3e38)))
        rows.append(np.full(cols, np.float32(-3e38)))
        r = np.full(cols, np.float32(3e38)); r[::2] = np.float32(-3e38); rows.append(r)
        rows.append(base())
        x = np.concatenate(rows)
        n = len(rows)
        a = Pair(x, [cols, n, 1, 1]).to(gpu)
        o = Pair(np.zeros(n, np.float32), [1, n, 1, 1]).to(gpu)
        assert eh.Kernel().process_event(eh.OpSumRows(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
        want = np.zeros(n, np.float32)
        assert orc.sum_rows(a.oview(), orc.view(want, o.ne)) == orc.OK
        got = o.result()
        assert np.isnan(want[0]) and np.isnan(want[3]) and want[2] == np.inf and want[4] == -np.inf
        assert_close_rel(got, want, 1e-5, f"sum_rows non-finite, {cols} columns",
                         atol=1e-12 * float(np.abs(x[np.isfinite(x)].astype(np.float64)).sum()))
        assert (np.isnan(got) == np.isnan(want)).all()
