"""GPU parity: emel-logits' native temperature/top-k sampler and candidate
validator through the C ABI, against the CPU oracle (oracle/
emel_oracle_sampler.c) on the same seeded inputs, bit for bit:

  - the final logits (the probabilities the softmax leaves in place; the
    sum is the reference's sequential f32 sum, reproduced exactly);
  - top_probabilities, top_indices and the first top_k sorted_indices
    (ties by ascending index on both sides);
  - selected token and score, the updated random state and the result
    guard's status.
NaN outputs compare as NaN (their payloads are not specified).
"""
import ctypes

import numpy as np
import pytest
import torch

import emel_hip as eh
import oracle as orc
from emel_hip.abi import CSampleRows

pytestmark = pytest.mark.gpu
M = 2147483647


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(both_nan | (a.view(np.uint32) == b.view(np.uint32))))


def oracle_rows(x, temperature, top_k, states):
    rows, card = x.shape
    out = []
    for r in range(rows):
        v = x[r].copy()
        srt = np.zeros(card, np.int32)
        tp = np.zeros(top_k, np.float32)
        ti = np.zeros(top_k, np.int32)
        rs = np.array([states[r]], np.uint32)
        sel = np.zeros(1, np.int32)
        sc = np.zeros(1, np.float32)
        st = orc.sample_temperature_top_k(card, temperature, top_k, v, srt, tp, ti, rs, sel, sc)
        out.append(dict(st=st, p=v, srt=srt[:top_k], tp=tp, ti=ti, rs=int(rs[0]), sel=int(sel[0]), sc=float(sc[0])))
    return out


def gpu_rows(gpu, x, temperature, top_k, states, pad=0, offset=0):
    """Runs every row of x in one batched call; rows `card + pad` apart,
    starting `offset` elements into the buffer (offset 1: rows not 16-byte
    aligned)."""
    rows, card = x.shape
    ld = card + pad
    buf = np.zeros(offset + rows * ld, np.float32)
    for r in range(rows):
        buf[offset + r * ld: offset + r * ld + card] = x[r]
    dbuf = torch.from_numpy(buf).to(gpu)
    logits = dbuf[offset:]
    srt = torch.full((rows * ld,), -5, dtype=torch.int32, device=gpu)
    tp = torch.full((rows * top_k,), 9.0, device=gpu)
    ti = torch.full((rows * top_k,), -9, dtype=torch.int32, device=gpu)
    sel = torch.full((rows,), -3, dtype=torch.int32, device=gpu)
    sc = torch.zeros(rows, device=gpu)
    status = torch.full((rows,), -1, dtype=torch.int32, device=gpu)
    rs = np.array(states, np.uint32)
    req = eh.SampleTemperatureTopK(card, temperature, top_k, logits, srt, tp, ti, rs, sel, sc, status_out=status)
    if rows == 1:
        st = eh.Status(eh.load().emel_sample_temperature_top_k(ctypes.byref(req.c()), None))
    else:
        cr = CSampleRows(rows, ld, ld, top_k)
        st = eh.Status(eh.load().emel_sample_temperature_top_k_rows(ctypes.byref(req.c()), ctypes.byref(cr), None))
    assert st == eh.Status.OK, eh.last_error()
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    out = []
    for r in range(rows):
        out.append(dict(p=lg[r * ld: r * ld + card], srt=srt.cpu().numpy()[r * ld: r * ld + top_k],
                        tp=tp.cpu().numpy()[r * top_k:(r + 1) * top_k], ti=ti.cpu().numpy()[r * top_k:(r + 1) * top_k],
                        rs=int(rs[r]), sel=int(sel[r].item()), sc=float(sc[r].item()), status=int(status[r].item())))
    return out


def check(gpu, x, temperature, top_k, states, **kw):
    want = oracle_rows(x, temperature, top_k, states)
    got = gpu_rows(gpu, x, temperature, top_k, states, **kw)
    for r, (g, w) in enumerate(zip(got, want)):
        assert same_bits(g["p"], w["p"]), (r, np.flatnonzero(g["p"].view(np.uint32) != w["p"].view(np.uint32))[:5])
        assert np.array_equal(g["ti"], w["ti"]), (r, g["ti"][:10], w["ti"][:10])
        assert np.array_equal(g["srt"], w["srt"]), r
        assert same_bits(g["tp"], w["tp"]), r
        assert g["rs"] == w["rs"] and g["sel"] == w["sel"], (r, g["sel"], w["sel"])
        assert same_bits(g["sc"], w["sc"]), (r, g["sc"], w["sc"])
        assert g["status"] == (0 if w["st"] == orc.OK else int(eh.Status.INVALID_REQUEST)), r
    return got, want


def test_reference_unit_case(gpu):
    # sampler/sm.rs:990-1019: logits [1, 3, 2], temperature 1, top_k 2, state 7
    got, want = check(gpu, np.array([[1.0, 3.0, 2.0]], np.float32), 1.0, 2, [7])
    assert 0 <= got[0]["sel"] < 3 and np.isfinite(got[0]["sc"])


def test_config5_vocabulary_batch(gpu):
    """64 sequences over a 151,936-token vocabulary (BASELINE config 5's
    logits), temperature 0.8, top_k 40."""
    g = np.random.Generator(np.random.PCG64(501))
    x = g.standard_normal((64, 151936), dtype=np.float64).astype(np.float32)
    states = [int(s) for s in g.integers(1, M, 64)]
    check(gpu, x, 0.8, 40, states)


@pytest.mark.parametrize("top_k,temperature", [(8192, 1.0), (1, 0.8), (4096, 0.5)])
def test_config5_vocabulary_large_and_single_top_k(gpu, top_k, temperature):
    """Full 151,936-token rows at the bench's second case (top_k 8192: the
    bucket path, its bracket's two lists and the grouped ranking) and at the
    extremes of top_k."""
    g = np.random.Generator(np.random.PCG64(502 + top_k))
    x = g.standard_normal((6, 151936), dtype=np.float64).astype(np.float32)
    check(gpu, x, temperature, top_k, [int(s) for s in g.integers(1, M, 6)])


@pytest.mark.parametrize("card,top_k,temperature,sigma", [
    (1, 1, 1.0, 1.0), (5, 5, 0.7, 1.0), (4097, 1, 1.0, 1.0), (4097, 4097, 1.0, 2.0), (100003, 64, 0.5, 1.0),
    (30000, 8192, 1.0, 1.0), (30000, 8193, 1.0, 1.0), (50000, 20000, 1.3, 1.0), (20000, 50, 0.02, 1.0),
    (20000, 3000, 0.02, 1.0), (9000, 100, 100.0, 1.0), (9000, 10, 1.0, 40.0)])
def test_sizes_and_temperatures(gpu, card, top_k, temperature, sigma):
    g = np.random.Generator(np.random.PCG64(card * 7 + top_k))
    rows = 3
    x = (g.standard_normal((rows, card)) * sigma).astype(np.float32)
    check(gpu, x, temperature, top_k, [int(s) for s in g.integers(1, M, rows)])


def test_many_rows_batch_the_ranking(gpu):
    """More rows than one ranking launch takes (the start states travel in
    the launch arguments, 512 rows a launch), for the in-LDS ranking and for
    the tiled merge (top_k > 8192)."""
    g = np.random.Generator(np.random.PCG64(80))
    x = g.standard_normal((1100, 3000)).astype(np.float32)
    check(gpu, x, 0.9, 25, [int(s) for s in g.integers(1, M, 1100)])
    x = g.standard_normal((600, 10000)).astype(np.float32)
    check(gpu, x, 1.0, 9000, [int(s) for s in g.integers(1, M, 600)])


def test_wide_chunks_take_the_three_pass_exact_sum(gpu):
    """300 rows of 60,000 logits make 9,216-column chunks, wider than the
    fused exp + prediction pass holds (8,192): the chunk maxima, the
    exponentials and the predictions then run as three kernels, the
    predictions from exact f64 chunk sums.  Narrower chunks (every other
    case here) take the fused pass and predict from approximate sums."""
    g = np.random.Generator(np.random.PCG64(81))
    x = g.standard_normal((300, 60000)).astype(np.float32)
    check(gpu, x, 0.8, 40, [int(s) for s in g.integers(1, M, 300)])


TIE_16_32 = np.float32(-6.978456974029541)  # glibc expf: 488.5 units of 2^-19, a tie while 16 <= S < 32
TIE_32_64 = np.float32(-6.953190326690674)  # 250.5 units of 2^-18, a tie while 32 <= S < 64


def one_tie_rows(g, rows, card):
    """Rows whose running sum passes 16 within the first 16 elements (logit
    0, e = 1), then grows by about 0.5 per 512-element sub-chunk (logits in
    [-7.6, -6.3]), with both tie logits at random places in every
    sub-chunk: in the binades [16, 32) and [32, 64) every sub-chunk then
    holds exactly one element that lands halfway between two units, whose
    rounding the prediction resolves from the parity of the units before
    it."""
    x = g.uniform(-7.6, -6.3, (rows, card)).astype(np.float32)
    x[:, :16] = 0.0
    for r in range(rows):
        for a0 in range(512, card, 512):
            n = min(512, card - a0)
            i, j = g.choice(n, 2, replace=False)
            x[r, a0 + i] = TIE_16_32
            x[r, a0 + j] = TIE_32_64
    return x


def test_tie_constants_are_ties():
    """The two logits' exponentials (host glibc expf, the function the GPU
    replica matches bit for bit) sit exactly halfway between units of their
    binade, and on whole units of the other one."""
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    a, b = np.float64(libm.expf(float(TIE_16_32))), np.float64(libm.expf(float(TIE_32_64)))
    assert np.ldexp(a, 19) % 1 == 0.5 and np.ldexp(a, 18) % 1 == 0.25
    assert np.ldexp(b, 18) % 1 == 0.5 and np.ldexp(b, 19) % 1 == 0.0


def test_one_tie_per_sub_chunk(gpu):
    """Sub-chunks predicted with exactly one tie, in both prediction paths:
    4 rows of 40,000 (1,024-column chunks, the fused pass, lanes holding two
    float4 of a wave-contiguous layout) and 300 rows of 60,000 (9,216-column
    chunks, the three-kernel path, eight consecutive elements per lane).  A
    wrong tie position or parity moves S by one unit and every p with it."""
    g = np.random.Generator(np.random.PCG64(82))
    x = one_tie_rows(g, 4, 40000)
    check(gpu, x, 1.0, 40, [3, 5, 7, 9])
    x = one_tie_rows(g, 300, 60000)
    check(gpu, x, 1.0, 40, [int(s) for s in g.integers(1, M, 300)])


def test_fast_candidate_list_and_its_fallback(gpu):
    """The list k_smp_div writes from the sub-chunk maxima's threshold, and
    the radix path it falls back to, in one batched call (top_k 40 over
    151,936 logits):
      row 0: N(0,1) on a 0.5 grid -- dozens of p ties at the top_k-th value,
             a few hundred candidates, ranked by index;
      row 1: all logits equal -- every element a candidate: past 8192 the
             radix path with its exact ties decides;
      row 2: N(0,1);
      row 3: 10,000 logits at 5.0 spread over the row -- the threshold is
             their p, more than 256 candidates in one workgroup."""
    g = np.random.Generator(np.random.PCG64(83))
    card = 151936
    x = g.standard_normal((4, card)).astype(np.float32)
    x[0] = np.round(x[0] * 2) / 2
    x[1] = 0.0
    x[3, g.choice(card, 10000, replace=False)] = 5.0
    check(gpu, x, 1.0, 40, [11, 13, 17, 19])


@pytest.mark.parametrize("rows,top_k", [(1, 8192), (2, 5000), (2, 300)])
def test_bucket_path_group_counts(gpu, rows, top_k):
    """The bucket path's ranking with 8 workgroups for one row (7 digit
    groups of A, then B), 6 for top_k 5000 and 2 for top_k 300 (just above
    config 5's 297 sub-chunks, so no fast list), on full 151,936-token rows."""
    g = np.random.Generator(np.random.PCG64(900 + top_k))
    x = (g.standard_normal((rows, 151936)) * 1.5).astype(np.float32)
    check(gpu, x, 0.9, top_k, [int(s) for s in g.integers(1, M, rows)])


def test_bucket_path_cases(gpu):
    """top_k 3000 over 40,000 logits (no fast list: the bucket path), one row
    per case of the first-digit split (A: keys above the threshold's first
    digit, B: keys at it):
      row 0: N(0,1);
      row 1: all logits equal -- B is the whole row, too long to list: the
             selection by scans of the row, ties by index;
      row 2: 20,000 logits at 1.0 under 1,000 larger ones -- B too long;
      row 3: 12,000 at 1.0 -- B listed, cut down to its exact threshold,
             where the ties exceed one workgroup's sort: scans again;
      row 4: 5,000 at 1.0 -- B cut to its exact threshold, the ties sorted
             by index;
      row 5: NaN -- every probability NaN, one key;
      row 6: logits spread over [-40, 40] -- B short, sorted uncut;
      row 7: 5,000 at the maximum -- A empty, B the top digit."""
    g = np.random.Generator(np.random.PCG64(84))
    card, rows = 40000, 8
    x = g.standard_normal((rows, card)).astype(np.float32)
    x[1] = 0.5
    for r, n in ((2, 20000), (3, 12000), (4, 5000)):
        x[r] -= 4.0
        cols = g.permutation(card)
        x[r, cols[:n]] = 1.0
        x[r, cols[n:n + 1000]] = 3.0 + g.random(1000).astype(np.float32)
    x[5, 123] = np.nan
    x[6] = np.linspace(-40, 40, card, dtype=np.float32)[g.permutation(card)]
    x[7] = np.minimum(x[7], 2.0)
    x[7, g.choice(card, 5000, replace=False)] = 3.0
    got, _ = check(gpu, x, 1.0, 3000, [int(s) for s in g.integers(1, M, rows)])
    assert got[5]["sel"] == -1


def test_unaligned_and_padded_rows(gpu):
    g = np.random.Generator(np.random.PCG64(77))
    x = g.standard_normal((4, 12345)).astype(np.float32)
    states = [3, 5, 7, 11]
    check(gpu, x, 0.9, 33, states, pad=3, offset=1)
    check(gpu, x, 0.9, 33, states, pad=5)


def test_ties_and_duplicate_logits(gpu):
    """Coarsely quantised logits: many equal probabilities, at the top and
    across the radix threshold; equal keys rank by ascending index."""
    g = np.random.Generator(np.random.PCG64(78))
    x = np.round(g.standard_normal((3, 50000)) * 4).astype(np.float32) / 4
    check(gpu, x, 1.0, 500, [17, 19, 23])
    check(gpu, x, 1.0, 9000, [17, 19, 23])


def test_nan_and_infinite_logits(gpu):
    card = 5000
    x = np.zeros((4, card), np.float32)
    x[0, 17] = np.nan                  # NaN row: every probability NaN, no race wins
    x[1, 3] = np.inf                   # +inf: inf - inf = NaN -> NaN row
    x[2, :] = -np.inf                  # all -inf: max -inf, NaN row
    x[3, 100] = -np.inf                # one -inf: probability 0
    got, want = check(gpu, x, 1.0, 7, [5, 6, 7, 8])
    assert got[0]["sel"] == -1 and got[0]["status"] == int(eh.Status.INVALID_REQUEST)
    assert got[3]["status"] == 0


def test_state_continues_across_calls(gpu):
    g = np.random.Generator(np.random.PCG64(79))
    x = g.standard_normal((1, 2000)).astype(np.float32)
    s = eh.Sampler()
    rs = np.array([12345], np.uint32)
    picks = []
    for _ in range(3):
        lg = torch.from_numpy(x[0].copy()).to(gpu)
        req = eh.SampleTemperatureTopK(2000, 1.0, 25, lg, torch.zeros(2000, dtype=torch.int32, device=gpu),
                                       torch.zeros(25, device=gpu), torch.zeros(25, dtype=torch.int32, device=gpu), rs,
                                       torch.zeros(1, dtype=torch.int32, device=gpu), torch.zeros(1, device=gpu))
        st, res = s.sample_temperature_top_k(req)
        assert st == eh.Status.OK
        picks.append(res)
    state = 12345
    for res in picks:
        w = oracle_rows(x, 1.0, 25, [state])[0]
        assert res[0] == w["sel"] and same_bits(res[1], w["sc"])
        state = w["rs"]
    assert int(rs[0]) == state


def test_validator_build(gpu):
    v = eh.Validator()
    cases = [np.array([1.0, 4.0, 2.5], np.float32), np.array([-0.0, 0.0, -1.0], np.float32),
             np.array([np.nan, 5.0, 1.0], np.float32),
             np.random.Generator(np.random.PCG64(80)).standard_normal(151936).astype(np.float32)]
    for x in cases:
        n = x.size
        ids = torch.full((n,), -1, dtype=torch.int32, device=gpu)
        sc = torch.full((n,), 99.0, device=gpu)
        b = eh.Build(torch.from_numpy(x).to(gpu), n, ids, sc, n)
        st, count = v.process_event(b)
        assert st == eh.Status.OK and count == n and b.error_out == 0
        wi = np.zeros(n, np.int32)
        ws = np.zeros(n, np.float32)
        cnt = np.zeros(1, np.int32)
        err = np.zeros(1, np.int32)
        assert orc.validator_build(x, n, wi, ws, n, cnt, err) == orc.OK
        assert np.array_equal(ids.cpu().numpy(), wi)
        assert same_bits(sc.cpu().numpy(), ws)
