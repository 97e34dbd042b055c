"""CPU: the oracle's restatement of emel-logits' sampler and validator
(oracle/emel_oracle_sampler.c) against the reference's own unit tests and
against independent computations:

  - sampler/sm.rs:990-1055 and tests/validator.rs (known answers, rejection
    without writes);
  - the Park-Miller minimal standard generator: from seed 1, the 10,000th
    state is 1043618065 (Park & Miller, CACM 31(10), 1988);
  - the softmax: glibc expf (called through ctypes), a numpy float32
    sequential cumsum for the sum, numpy float32 division -- bit for bit;
    and a float64 softmax within 1e-5 relative;
  - the ranking: numpy's stable argsort of -p (ties by ascending index);
  - the race: glibc logf through ctypes and numpy float32 division, the
    first maximal race winning.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

import oracle as orc

LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
LIBM.expf.restype = ctypes.c_float
LIBM.expf.argtypes = [ctypes.c_float]
LIBM.logf.restype = ctypes.c_float
LIBM.logf.argtypes = [ctypes.c_float]
M = 2147483647


def run(logits, temperature, top_k, state, sorted_len=None, tp_len=None):
    card = logits.size
    x = logits.astype(np.float32).copy()
    srt = np.full(card if sorted_len is None else sorted_len, -7, np.int32)
    tp = np.full(top_k if tp_len is None else tp_len, 99.0, np.float32)
    ti = np.full(top_k if tp_len is None else tp_len, -9, np.int32)
    rs = np.array([state], np.uint32)
    sel = np.array([11], np.int32)
    sc = np.array([12.0], np.float32)
    st = orc.sample_temperature_top_k(card, temperature, top_k, x, srt, tp, ti, rs, sel, sc)
    return st, x, srt, tp, ti, int(rs[0]), int(sel[0]), float(sc[0])


def test_reference_native_temperature_top_k_returns_finite_result():
    # sampler/sm.rs:990-1019
    st, _, _, _, _, _, sel, sc = run(np.array([1.0, 3.0, 2.0], np.float32), 1.0, 2, 7)
    assert st == orc.OK
    assert 0 <= sel < 3 and np.isfinite(sc)


def test_reference_invalid_temperature_capacity_fails_before_writes():
    # sampler/sm.rs:1021-1055: sorted scratch shorter than card
    logits = np.array([1.0, 3.0, 2.0], np.float32)
    st, x, srt, _, _, rs, sel, sc = run(logits, 1.0, 2, 7, sorted_len=2)
    assert st == orc.INVALID_REQUEST
    assert x.view(np.uint32).tolist() == logits.view(np.uint32).tolist()
    assert rs == 7 and sel == 11 and np.float32(sc).view(np.uint32) == np.float32(12.0).view(np.uint32)


@pytest.mark.parametrize("case", [
    dict(temperature=0.0), dict(temperature=-1.0), dict(temperature=float("inf")), dict(temperature=float("nan")),
    dict(top_k=0), dict(top_k=4), dict(state=0), dict(state=M), dict(state=2 * M), dict(tp_len=1),
])
def test_guard_rejections_write_nothing(case):
    args = dict(temperature=1.0, top_k=2, state=7)
    args.update(case)
    tp_len = args.pop("tp_len", None)
    logits = np.array([1.0, 3.0, 2.0], np.float32)
    st, x, srt, tp, _, rs, sel, _ = run(logits, args["temperature"], args["top_k"], args["state"], tp_len=tp_len)
    assert st == orc.INVALID_REQUEST
    assert np.array_equal(x, logits) and (srt == -7).all() and (tp == 99.0).all()
    assert rs == args["state"] and sel == 11


def test_park_miller_minimal_standard_check_value():
    s = 1
    for _ in range(10_000):
        s = orc.park_miller_next(s)
    assert s == 1043618065


def glibc_softmax(v):
    m = np.float32(-np.inf)
    for a in v:
        if a > m:
            m = a
    e = np.array([LIBM.expf(float(np.float32(a - m))) for a in v], np.float32)
    total = np.cumsum(e, dtype=np.float32)[-1]  # sequential float32 accumulation
    return e / total, total


@pytest.mark.parametrize("seed,card,sigma", [(1, 257, 1.0), (2, 3000, 3.0), (3, 5000, 0.01), (4, 40, 30.0)])
def test_softmax_bits_against_glibc_and_numpy(seed, card, sigma):
    g = np.random.Generator(np.random.PCG64(seed))
    v = (g.standard_normal(card) * sigma).astype(np.float32)
    got = v.copy()
    total = orc.sampler_softmax(got)
    want, want_total = glibc_softmax(v)
    assert np.float32(total).view(np.uint32) == want_total.view(np.uint32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    exact = np.exp(v.astype(np.float64) - v.max())
    exact /= exact.sum()
    nz = exact > 1e-30
    assert np.max(np.abs(got[nz] - exact[nz]) / exact[nz]) < 1e-5


def test_sequential_sum_is_not_a_tree_sum():
    """The restatement keeps the reference's sequential f32 rounding: for a
    long vocabulary row it differs from a float64 sum (and so would any
    reordered sum), which is why the GPU must reproduce it exactly."""
    g = np.random.Generator(np.random.PCG64(9))
    v = g.standard_normal(151936).astype(np.float32)
    total = orc.sampler_softmax(v.copy())
    e = np.exp(v.astype(np.float64) - v.max())
    assert np.float32(total) != np.float32(e.sum())
    assert abs(total - e.sum()) / e.sum() < 1e-3


@pytest.mark.parametrize("seed,card,top_k,temperature", [(5, 1000, 40, 0.8), (6, 4096, 1, 1.0), (7, 300, 300, 2.0),
                                                          (8, 151, 17, 0.05)])
def test_rank_and_select_against_independent_restatement(seed, card, top_k, temperature):
    g = np.random.Generator(np.random.PCG64(seed))
    logits = g.standard_normal(card).astype(np.float32)
    state0 = int(g.integers(1, M))
    st, x, srt, tp, ti, rs, sel, sc = run(logits, temperature, top_k, state0)
    assert st == orc.OK
    v = logits * np.float32(np.float32(1.0) / np.float32(temperature))
    p, _ = glibc_softmax(v)
    assert np.array_equal(x.view(np.uint32), p.view(np.uint32))
    order = np.argsort(-p, kind="stable")
    assert np.array_equal(ti, order[:top_k]) and np.array_equal(srt, order)
    assert np.array_equal(tp.view(np.uint32), p[order[:top_k]].view(np.uint32))
    s, best, pick = state0, np.float32(-np.inf), -1
    for j in range(top_k):
        s = s * 16807 % M
        u = np.float32(np.float32(s) / np.float32(M))
        race = np.float32(tp[j] / np.float32(-LIBM.logf(float(u))))
        if race > best:
            best, pick = race, int(ti[j])
    assert rs == s and sel == pick and np.float32(sc).view(np.uint32) == best.view(np.uint32)


def test_ties_rank_by_ascending_index():
    logits = np.array([0.5, 2.0, 2.0, -1.0, 2.0, 0.5], np.float32)
    st, _, srt, _, ti, _, _, _ = run(logits, 1.0, 4, 12345)
    assert st == orc.OK
    assert ti.tolist() == [1, 2, 4, 0] and srt.tolist() == [1, 2, 4, 0, 5, 3]


def test_result_guard_failure_still_writes_outputs():
    # every probability 0 except NaN ones: every race is NaN or 0/x = 0 ...
    # a NaN logit makes the whole row NaN (the sum is NaN): no race > -inf
    logits = np.array([1.0, np.nan, 2.0], np.float32)
    st, x, _, _, _, rs, sel, sc = run(logits, 1.0, 2, 7)
    assert st == orc.INVALID_REQUEST
    assert np.isnan(x).all()
    assert sel == -1 and sc == -np.inf and rs == 7 * 16807 * 16807 % M


def test_reference_validator_build_normalizes_logits():
    # tests/validator.rs: build_normalizes_logits
    logits = np.array([1.0, 4.0, 2.5], np.float32)
    ids = np.full(3, -1, np.int32)
    scores = np.full(3, 99.0, np.float32)
    count = np.array([-1], np.int32)
    err = np.array([3], np.int32)
    assert orc.validator_build(logits, 3, ids, scores, 3, count, err) == orc.OK
    assert ids.tolist() == [0, 1, 2] and scores.tolist() == [-3.0, 0.0, -1.5]
    assert count[0] == 3 and err[0] == 0


@pytest.mark.parametrize("vocab,capacity", [(0, 2), (2, 1), (-1, 2), (3, 3)])
def test_reference_validator_rejects_invalid_sizes_and_resets_outputs(vocab, capacity):
    # tests/validator.rs: build_rejects_invalid_sizes_and_resets_outputs
    logits = np.array([1.0, 2.0], np.float32)
    ids = np.full(2, 7, np.int32)
    scores = np.full(2, 8.0, np.float32)
    count = np.array([9], np.int32)
    err = np.array([2], np.int32)
    assert orc.validator_build(logits, vocab, ids, scores, capacity, count, err) == orc.INVALID_REQUEST
    assert count[0] == 0 and err[0] == 1


def test_validator_max_is_the_first_maximal_element():
    # strict > from logits[0]: -0.0 stays the maximum over a later +0.0, and a
    # leading NaN stays the maximum (every score NaN)
    logits = np.array([-0.0, 0.0, -1.0], np.float32)
    ids = np.zeros(3, np.int32)
    scores = np.zeros(3, np.float32)
    count = np.zeros(1, np.int32)
    err = np.zeros(1, np.int32)
    assert orc.validator_build(logits, 3, ids, scores, 3, count, err) == orc.OK
    assert scores.view(np.uint32).tolist() == np.array([0.0, 0.0, -1.0], np.float32).view(np.uint32).tolist()
    logits = np.array([np.nan, 5.0], np.float32)
    assert orc.validator_build(logits, 2, ids[:2].copy(), s2 := np.zeros(2, np.float32), 2, count, err) == orc.OK
    assert np.isnan(s2).all()
