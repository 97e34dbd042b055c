"""GPU parity: rms_norm (+weight), norm and soft_max vs the CPU oracle.

The reference accumulates these row sums sequentially in f64 (rms_norm,
norm, dense soft_max); the GPU sums the same f64 terms in a tree, so an f32
result can differ only when the f64 sum lands next to an f32 rounding
boundary.  The tolerance is BASELINE's: 1e-5 relative.  The strided
soft_max keeps the reference's sequential f32 sum and is compared
bit-exactly.
"""
import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from helpers import Pair, assert_bits_equal, assert_close_rel, normal, uniform

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def outlier_rows(x, cols, rows, seed, frac=0.01, factor=100.0):
    g = np.random.Generator(np.random.PCG64(seed))
    picked = g.choice(rows, max(1, int(rows * frac)), replace=False)
    x = x.reshape(rows, cols).copy()
    x[picked] *= np.float32(factor)
    return x.reshape(-1)


# (2048, 2048), (8192, 1536), (4096, 4096), (2048, 1536): one wave per row; (4096, 1535), (2048, 4097):
# just outside the row range
@pytest.mark.parametrize("cols,rows", [(4096, 2048), (4096, 3), (1, 5), (3, 7), (64, 64), (1000, 9),
                                       (8192, 4), (20000, 3), (2048, 2048), (8192, 1536), (4096, 4096),
                                       (4096, 1535), (2048, 1536), (2048, 4097)])
def test_rms_norm(gpu, cols, rows):
    x = outlier_rows(normal(101 + cols, cols * rows), cols, rows, 7)
    a = Pair(x, [cols, rows, 1, 1]).to(gpu)
    o = Pair(np.zeros_like(x), [cols, rows, 1, 1]).to(gpu)
    assert eh.Kernel().process_event(eh.OpRmsNorm(a.pview(), o.pview(mut=True), 1e-5)) == eh.Status.OK, eh.last_error()
    want = np.zeros_like(x)
    assert orc.rms_norm(a.oview(), orc.view(want, o.ne), 1e-5) == orc.OK
    got = o.result()
    assert_close_rel(got, want, RTOL, "rms_norm")
    # informational: the tree-ordered f64 sum almost always rounds alike
    exact = (got.view(np.uint32) == want.view(np.uint32)).mean()
    assert exact > 0.99, f"only {exact:.4%} bit-exact"


@pytest.mark.parametrize("cols,rows", [(4096, 2048), (2048, 1600), (8192, 2048), (4096, 1024)])
def test_rms_norm_mul(gpu, cols, rows):
    x = outlier_rows(normal(111, cols * rows), cols, rows, 8)
    w = uniform(112, cols, 0.5, 1.5)
    a = Pair(x, [cols, rows, 1, 1]).to(gpu)
    wp = Pair(w, [cols, 1, 1, 1]).to(gpu)
    o = Pair(np.zeros_like(x), [cols, rows, 1, 1]).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpRmsNormMul(a.pview(), wp.pview(), o.pview(mut=True), 1e-5)) == eh.Status.OK
    want = np.zeros_like(x)
    assert orc.rms_norm_mul(a.oview(), wp.oview(), orc.view(want, o.ne), 1e-5) == orc.OK
    assert_close_rel(o.result(), want, RTOL, "rms_norm_mul")
    # fused == rms_norm then OpMulBroadcastRow on the GPU, bit for bit
    t = Pair(np.zeros_like(x), o.ne).to(gpu)
    o2 = Pair(np.zeros_like(x), o.ne).to(gpu)
    assert k.process_event(eh.OpRmsNorm(a.pview(), t.pview(mut=True), 1e-5)) == eh.Status.OK
    assert k.process_event(eh.OpMulBroadcastRow(t.pview(), wp.pview(), o2.pview(mut=True))) == eh.Status.OK
    assert_bits_equal(o.result(), o2.result(), "fused vs composed rms_norm * w")


def test_rms_norm_strided_and_implicit(gpu):
    cols, rows = 300, 11
    # rows padded to 320 floats, dim 0 stride 8 bytes (every other float)
    st = Pair(normal(121, 2 * 320 * rows), [cols // 2, rows, 1, 1], [8, 4 * 320, 4 * 320 * rows, 4 * 320 * rows]).to(gpu)
    o = Pair(np.zeros(cols // 2 * rows, np.float32), [cols // 2, rows, 1, 1]).to(gpu)
    assert eh.Kernel().process_event(eh.OpRmsNorm(st.pview(), o.pview(mut=True), 0.5)) == eh.Status.OK, eh.last_error()
    want = np.zeros(cols // 2 * rows, np.float32)
    assert orc.rms_norm(st.oview(), orc.view(want, o.ne), 0.5) == orc.OK
    assert_close_rel(o.result(), want, RTOL, "strided rms_norm")
    im = Pair(normal(122, cols * rows), [cols, rows, 1, 1], [0, 0, 0, 0]).to(gpu)
    o = Pair(np.zeros(cols * rows, np.float32), [cols, rows, 1, 1], [0, 0, 0, 0]).to(gpu)
    assert eh.Kernel().process_event(eh.OpRmsNorm(im.pview(), o.pview(mut=True), 1.0)) == eh.Status.OK
    want = np.zeros(cols * rows, np.float32)
    assert orc.rms_norm(im.oview(), orc.view(want, o.ne, o.nb), 1.0) == orc.OK
    assert_close_rel(o.result(), want, RTOL, "implicit rms_norm")


@pytest.mark.parametrize("op", ["rms_norm", "norm"])
def test_norm_rows_padded_pitch(gpu, op):
    """Rows 8 floats apart (a 16-byte-aligned pitch that is not the width) in the one-wave-per-row range."""
    cols, rows = 4096, 2048
    x = outlier_rows(normal(151, cols * rows, 2.0), cols, rows, 9) + np.float32(0.5)
    a = padded_pair(x, cols, rows, 8).to(gpu)
    o = Pair(np.zeros(cols * rows, np.float32), [cols, rows, 1, 1]).to(gpu)
    ev = eh.OpRmsNorm if op == "rms_norm" else eh.OpNorm
    assert eh.Kernel().process_event(ev(a.pview(), o.pview(mut=True), 1e-5)) == eh.Status.OK, eh.last_error()
    want = np.zeros(cols * rows, np.float32)
    fn = orc.rms_norm if op == "rms_norm" else orc.norm
    assert fn(a.oview(), orc.view(want, o.ne), 1e-5) == orc.OK
    assert_close_rel(o.result(), want, RTOL, f"{op} with a padded row pitch", atol=1e-6)


@pytest.mark.parametrize("cols,rows", [(4096, 64), (7, 9), (10000, 5), (4096, 2048), (2048, 3000), (8192, 1600)])
def test_norm(gpu, cols, rows):
    x = normal(131, cols * rows, 3.0) + np.float32(2.0)
    a = Pair(x, [cols, rows, 1, 1]).to(gpu)
    o = Pair(np.zeros_like(x), a.ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpNorm(a.pview(), o.pview(mut=True), 1e-5)) == eh.Status.OK
    want = np.zeros_like(x)
    assert orc.norm(a.oview(), orc.view(want, a.ne), 1e-5) == orc.OK
    assert_close_rel(o.result(), want, RTOL, "norm", atol=1e-6)


@pytest.mark.parametrize("cols,rows", [(4096, 256), (3, 2), (5, 17), (151936, 2), (1, 4)])
def test_soft_max_dense(gpu, cols, rows):
    x = normal(141 + cols, cols * rows, 2.0)
    a = Pair(x, [cols, rows, 1, 1]).to(gpu)
    o = Pair(np.zeros_like(x), a.ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpSoftMax(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = np.zeros_like(x)
    assert orc.soft_max(a.oview(), orc.view(want, a.ne)) == orc.OK
    assert_close_rel(o.result(), want, RTOL, "soft_max")


def test_soft_max_strided_is_bit_exact(gpu):
    cols, rows = 513, 37
    # dim 0 stride 8 bytes: not dense, so the reference sums in sequential f32
    a = Pair(normal(151, 2 * cols * rows, 3.0), [cols, rows, 1, 1],
             [8, 8 * cols, 8 * cols * rows, 8 * cols * rows]).to(gpu)
    o = Pair(np.zeros(cols * rows, np.float32), [cols, rows, 1, 1]).to(gpu)
    assert eh.Kernel().process_event(eh.OpSoftMax(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = np.zeros(cols * rows, np.float32)
    assert orc.soft_max(a.oview(), orc.view(want, o.ne)) == orc.OK
    assert_bits_equal(o.result(), want, "strided soft_max")


# ---- strided soft_max: the exact sequential f32 row sum -------------------------
#
# Any layout that is not dense row-major makes the reference sum each row's
# exponentials one by one in f32 (reductions.rs:603-638).  The GPU reproduces
# that sum exactly (a lane per row up to 64 columns, a workgroup per row with
# the binade walk above that); every case is bit-exact against the oracle.

def padded_pair(x, cols, rows, pad):
    """Rows of `cols` values `pad` floats apart: not dense."""
    buf = np.zeros((rows, cols + pad), np.float32)
    buf[:, :cols] = x.reshape(rows, cols)
    pitch = 4 * (cols + pad)
    return Pair(buf.reshape(-1), [cols, rows, 1, 1], [4, pitch, pitch * rows, pitch * rows])


def strided_soft_max(gpu, a, out_ne):
    n = int(np.prod(a.ne))
    o = Pair(np.zeros(n, np.float32), out_ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpSoftMax(a.to(gpu).pview(), o.pview(mut=True))) == eh.Status.OK, \
        eh.last_error()
    want = np.zeros(n, np.float32)
    assert orc.soft_max(a.oview(), orc.view(want, o.ne, o.nb)) == orc.OK
    return o.result(), want


@pytest.mark.parametrize("cols,rows", [(4096, 512), (65, 40), (511, 7), (512, 9), (513, 5), (1024, 33),
                                       (2048, 7), (2049, 3), (4097, 3), (20000, 4), (100000, 2), (64, 300),
                                       (1025, 3), (8192, 3), (8193, 2), (16384, 2), (16385, 2), (32768, 1)])
def test_soft_max_strided_rows_bit_exact(gpu, cols, rows):
    x = normal(700 + cols, cols * rows, 3.0)
    got, want = strided_soft_max(gpu, padded_pair(x, cols, rows, 3), [cols, rows, 1, 1])
    assert_bits_equal(got, want, f"strided soft_max {cols}x{rows}")


def test_soft_max_strided_transposed_and_reshaped_dst(gpu):
    cols, rows = 3000, 6
    x = normal(710, cols * rows, 2.0)
    # column-major storage: dim 0 has stride rows * 4 bytes
    a = Pair(x.reshape(cols, rows).copy().reshape(-1), [cols, rows, 1, 1], [4 * rows, 4, 4 * cols * rows,
                                                                           4 * cols * rows])
    got, want = strided_soft_max(gpu, a, [cols, rows, 1, 1])
    assert_bits_equal(got, want, "transposed soft_max")
    # a dst of the same count but another shape: its ordinals are decoded per element
    got, want = strided_soft_max(gpu, padded_pair(x, cols, rows, 1), [rows * 2, cols // 2, 1, 1])
    assert_bits_equal(got, want, "soft_max into a reshaped dst")


@pytest.mark.parametrize("cols", [4096, 20000, 300, 65, 37])
def test_soft_max_strided_non_finite(gpu, cols):
    x, rows = special_rows(cols, 720 + cols)
    got, want = strided_soft_max(gpu, padded_pair(x, cols, rows, 2), [cols, rows, 1, 1])
    assert np.isnan(want.reshape(rows, cols)[0]).all()
    assert_bits_equal(got, want, f"strided soft_max non-finite, {cols} columns")


# x for which glibc's expf is exactly k/8, so that, once the running sum has
# a spacing of 1/4 (from 2^21 on), odd multiples of 1/8 are rounding ties
# (found by searching the float neighbours of log(k/8) against glibc).
DYADIC_EXP = {1.0: 0.0, 0.875: -0.133531391620636, 0.75: -0.28768208622932434, 0.625: -0.4700036346912384,
              0.5: -0.6931471824645996, 0.375: -0.9808292388916016, 0.25: -1.3862943649291992,
              0.125: -2.079441547393799}


def test_soft_max_strided_ties_and_saturation(gpu):
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype, libm.expf.argtypes = ctypes.c_float, [ctypes.c_float]
    for value, arg in DYADIC_EXP.items():
        assert libm.expf(arg) == value
    g = np.random.Generator(np.random.PCG64(730))
    cols = (1 << 21) + (1 << 18)
    keys = np.array(list(DYADIC_EXP.values()), np.float32)
    x = np.where(g.random(cols) < 0.9, np.float32(0.0), keys[g.integers(0, len(keys), cols)]).astype(np.float32)
    got, want = strided_soft_max(gpu, padded_pair(x, cols, 1, 1), [cols, 1, 1, 1])
    assert_bits_equal(got, want, "soft_max with rounding ties")
    # 2^24 ones saturate the f32 sum: every later +1 is a tie that rounds back
    cols = (1 << 24) + 4096
    got, want = strided_soft_max(gpu, padded_pair(np.zeros(cols, np.float32), cols, 1, 1), [cols, 1, 1, 1])
    assert_bits_equal(got, want, "soft_max with a saturated sum")
    assert got[0] == np.float32(2.0 ** -24)


def exp_preimage(libm, value):
    """A float32 x with glibc's expf(x) == value exactly, by walking the float neighbours of log(value)."""
    x = np.float32(np.log(value))
    for direction in (np.float32(np.inf), np.float32(-np.inf)):
        y = x
        for _ in range(4096):
            if libm.expf(float(y)) == value:
                return y
            y = np.nextafter(y, direction)
    raise AssertionError(f"no float32 x with expf(x) == {value}")


def sequential_ties(e):
    """Additions of the sequential float32 sum of e whose exact result is a rounding tie."""
    s = np.concatenate([[np.float32(0.0)], np.cumsum(e, dtype=np.float32)[:-1]]).astype(np.float64)
    exact = s + e.astype(np.float64)
    ulp = np.ldexp(1.0, np.frexp(exact)[1] - 24)
    return int(np.count_nonzero((exact > 0) & (np.mod(exact, ulp) == ulp / 2)))


@pytest.mark.parametrize("cols", [512, 1024, 2048, 4096, 8192, 20000])
def test_soft_max_strided_sparse_ties(gpu, cols):
    """Rows of ones (x = 0) with a few addends 1 - 2^(k - 24): once the running sum passes 2^k they are
    exact rounding ties, a handful per segment, next to runs of addends that are not."""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype, libm.expf.argtypes = ctypes.c_float, [ctypes.c_float]
    top = int(np.log2(cols))
    keys = np.array([exp_preimage(libm, 1.0 - 2.0 ** (k - 24)) for k in range(top - 3, top + 1)], np.float32)
    g = np.random.Generator(np.random.PCG64(740 + cols))
    rows = 6
    x = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        density = (1 / 64, 1 / 16, 1 / 4, 1 / 200, 1 / 32, 1 / 8)[r]
        pick = g.random(cols) < density
        x[r, pick] = keys[g.integers(0, len(keys), int(pick.sum()))]
    e = np.ones((rows, cols), np.float32)  # the row max is 0: expf(x - 0)
    e[x != 0] = np.array([libm.expf(float(v)) for v in x[x != 0]], np.float32)
    assert sum(sequential_ties(e[r]) for r in range(rows)) >= rows * 4
    got, want = strided_soft_max(gpu, padded_pair(x.reshape(-1), cols, rows, 2), [cols, rows, 1, 1])
    assert_bits_equal(got, want, f"strided soft_max with sparse ties, {cols} columns")


def causal_mask(nkv, nq):
    k = np.arange(nkv)[None, :]
    q = np.arange(nq)[:, None]
    return np.where(k <= q + (nkv - nq), np.float16(0.0), np.float16(-np.inf)).astype(np.float16).reshape(-1)


@pytest.mark.parametrize("nkv,nq,nh", [(4096, 512, 32), (256, 64, 4), (36, 5, 3), (4096, 1, 2)])
def test_soft_max_ext_causal(gpu, nkv, nq, nh):
    x = normal(161, nkv * nq * nh, 2.0)  # N(0, 4)
    scale = float(np.float32(1.0 / np.sqrt(128.0)))
    a = Pair(x, [nkv, nq, nh, 1]).to(gpu)
    m = Pair(causal_mask(nkv, nq).view(np.uint16), [nkv, nq, 1, 1], dtype=orc.F16).to(gpu)
    o = Pair(np.zeros_like(x), a.ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpSoftMaxExt(a.pview(), m.pview(), scale, o.pview(mut=True))) == eh.Status.OK, \
        eh.last_error()
    want = np.zeros_like(x)
    assert orc.soft_max_ext(a.oview(), m.oview(), scale, orc.view(want, a.ne)) == orc.OK
    got = o.result()
    assert_close_rel(got, want, RTOL, "soft_max_ext")
    rows = got.reshape(-1, nkv).astype(np.float64).sum(axis=1)
    assert np.abs(rows - 1.0).max() < 1e-5


@pytest.mark.parametrize("nkv,nq,nh,n3,m2,m3", [
    (20000, 3, 2, 1, 1, 1),    # rows wider than the registers hold: the streamed passes
    (40000, 2, 2, 1, 2, 1),    # streamed, one mask per head
    (4096, 8, 4, 1, 4, 1),     # config 4's width, one mask per head
    (1024, 4, 6, 2, 3, 2),     # mask broadcast over dims 2 and 3 (m2 | ne2, m3 | ne3)
])
def test_soft_max_ext_wide_rows_and_broadcast_masks(gpu, nkv, nq, nh, n3, m2, m3):
    x = normal(191 + nkv + m2, nkv * nq * nh * n3, 2.0)
    g = np.random.Generator(np.random.PCG64(192 + nkv))
    mask = (g.standard_normal(nkv * nq * m2 * m3) * 2).astype(np.float16)
    mask[g.random(mask.size) < 0.3] = np.float16(-np.inf)
    mask.reshape(-1, nkv)[:, 0] = 0  # keep every row alive
    a = Pair(x, [nkv, nq, nh, n3]).to(gpu)
    m = Pair(mask.view(np.uint16), [nkv, nq, m2, m3], dtype=orc.F16).to(gpu)
    o = Pair(np.zeros_like(x), a.ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpSoftMaxExt(a.pview(), m.pview(), 0.5, o.pview(mut=True))) == eh.Status.OK, \
        eh.last_error()
    want = np.zeros_like(x)
    assert orc.soft_max_ext(a.oview(), m.oview(), 0.5, orc.view(want, a.ne)) == orc.OK
    assert_close_rel(o.result(), want, RTOL, "soft_max_ext wide / broadcast mask")


def test_soft_max_ext_reduces_to_soft_max(gpu):
    # zero mask and scale 1 must give OpSoftMax's bits exactly
    nkv, nq, nh = 1024, 16, 4
    x = normal(171, nkv * nq * nh, 2.0)
    a = Pair(x, [nkv, nq, nh, 1]).to(gpu)
    m = Pair(np.zeros(nkv * nq, np.uint16), [nkv, nq, 1, 1], dtype=orc.F16).to(gpu)
    o1 = Pair(np.zeros_like(x), a.ne).to(gpu)
    o2 = Pair(np.zeros_like(x), a.ne).to(gpu)
    k = eh.Kernel()
    assert k.process_event(eh.OpSoftMaxExt(a.pview(), m.pview(), 1.0, o1.pview(mut=True))) == eh.Status.OK
    assert k.process_event(eh.OpSoftMax(a.pview(), o2.pview(mut=True))) == eh.Status.OK
    assert_bits_equal(o1.result(), o2.result(), "ext(zero mask, scale 1) vs soft_max")


def test_soft_max_ext_general_path(gpu):
    # ncols % 4 != 0 and a per-head mask (m2 == nh): the non-vectorized kernel
    nkv, nq, nh = 37, 6, 4
    x = normal(181, nkv * nq * nh, 2.0)
    g = np.random.Generator(np.random.PCG64(182))
    mask = g.standard_normal(nkv * nq * nh).astype(np.float16)
    mask[g.random(mask.size) < 0.2] = np.float16(-np.inf)
    mask.reshape(-1, nkv)[:, 0] = 0  # keep every row alive
    a = Pair(x, [nkv, nq, nh, 1]).to(gpu)
    m = Pair(mask.view(np.uint16), [nkv, nq, nh, 1], dtype=orc.F16).to(gpu)
    o = Pair(np.zeros_like(x), a.ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpSoftMaxExt(a.pview(), m.pview(), 0.75, o.pview(mut=True))) == eh.Status.OK
    want = np.zeros_like(x)
    assert orc.soft_max_ext(a.oview(), m.oview(), 0.75, orc.view(want, a.ne)) == orc.OK
    assert_close_rel(o.result(), want, RTOL, "soft_max_ext general")


def test_rows_in_place(gpu):
    cols, rows = 4096, 16
    x = normal(191, cols * rows)
    for ev, fn in ((lambda v, o: eh.OpRmsNorm(v, o, 1e-5), lambda a, o: orc.rms_norm(a, o, 1e-5)),
                   (eh.OpSoftMax, orc.soft_max)):
        a = Pair(x, [cols, rows, 1, 1]).to(gpu)
        assert eh.Kernel().process_event(ev(a.pview(), a.pview(mut=True))) == eh.Status.OK
        want = x.copy()
        assert fn(orc.view(x, a.ne), orc.view(want, a.ne)) == orc.OK
        assert_close_rel(a.result(), want, RTOL, "in place")


# ---- non-finite inputs --------------------------------------------------------
#
# The reference seeds a row's max with column 0 and scans with a strict >
# (reductions.rs:565-601), so a NaN anywhere in a row, or a +inf, makes every
# exp(x - max) of that row NaN or the sum NaN: the whole row is NaN.  A row
# that is entirely -inf has max -inf, and exp(-inf - -inf) = exp(NaN) makes
# it NaN too.  -inf entries among finite ones give exp(-inf) = 0.  The GPU's
# max ignores NaN; the rows still agree because the NaN reaches the sum.

def special_rows(cols, seed):
    """One row per case, N(0, 4) elsewhere."""
    g = np.random.Generator(np.random.PCG64(seed))
    rows = []
    def base():
        return (g.standard_normal(cols) * 2).astype(np.float32)
    r = base(); r[0] = np.nan; rows.append(r)                           # NaN at column 0
    r = base(); r[cols // 2] = np.nan; rows.append(r)                   # NaN mid-row
    r = base(); r[-1] = np.nan; r[0] = -np.inf; rows.append(r)          # NaN last, -inf first
    r = base(); r[cols // 3] = np.inf; rows.append(r)                   # one +inf
    r = base(); r[0] = np.inf; r[-1] = np.inf; rows.append(r)           # two +inf
    r = base(); r[g.random(cols) < 0.5] = -np.inf; r[cols // 2] = 1.0; rows.append(r)  # -inf among finite
    rows.append(np.full(cols, -np.inf, np.float32))                     # all -inf
    r = base(); r[1 % cols] = np.inf; r[0] = -np.inf; rows.append(r)    # +inf and -inf
    r = base(); r[:] = np.float32(3e38); rows.append(r)                 # large equal values
    r = base(); r[0] = np.float32(1e-45); rows.append(r)                # a subnormal
    rows.append(base())                                                 # ordinary row
    return np.concatenate(rows).astype(np.float32), len(rows)


@pytest.mark.parametrize("cols", [4096, 256, 20000, 37, 1])
def test_soft_max_non_finite(gpu, cols):
    # 4096: one workgroup per row in registers; 256: one wave per row;
    # 20000: streamed passes; 37: the general (unvectorized) kernel; 1: one column
    x, rows = special_rows(cols, 401 + cols)
    a = Pair(x, [cols, rows, 1, 1]).to(gpu)
    o = Pair(np.zeros_like(x), a.ne).to(gpu)
    assert eh.Kernel().process_event(eh.OpSoftMax(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
    want = np.zeros_like(x)
    assert orc.soft_max(a.oview(), orc.view(want, a.ne)) == orc.OK
    got = o.result()
    assert np.isnan(want.reshape(rows, cols)[0]).all()  # the rule above, as the oracle states it
    assert_close_rel(got, want, RTOL, f"soft_max non-finite, {cols} columns")
    assert (np.isnan(got) == np.isnan(want)).all()


@pytest.mark.parametrize("nkv,nq,nh", [(4096, 8, 2), (512, 16, 3), (20000, 6, 2), (37, 6, 2)])
def test_soft_max_ext_fully_masked_and_non_finite(gpu, nkv, nq, nh):
    g = np.random.Generator(np.random.PCG64(411 + nkv))
    x = (g.standard_normal(nkv * nq * nh) * 2).astype(np.float32)
    xr = x.reshape(nh, nq, nkv)
    xr[0, 1, nkv // 2] = np.nan        # NaN score
    xr[1, 2, 0] = np.inf               # +inf score at column 0
    xr[0, 3, -1] = -np.inf             # -inf score
    mask = np.zeros((nq, nkv), np.float16)
    mask[g.random(mask.shape) < 0.4] = np.float16(-np.inf)
    mask[0, :] = np.float16(-np.inf)   # query row 0 fully masked in every head
    mask[4, 0] = np.float16(np.inf)    # +inf in the mask
    mask[5, :] = np.float16(65504.0)   # largest finite half
    a = Pair(x, [nkv, nq, nh, 1]).to(gpu)
    m = Pair(mask.reshape(-1).view(np.uint16), [nkv, nq, 1, 1], dtype=orc.F16).to(gpu)
    o = Pair(np.zeros_like(x), a.ne).to(gpu)
    scale = float(np.float32(1.0 / np.sqrt(128.0)))
    assert eh.Kernel().process_event(eh.OpSoftMaxExt(a.pview(), m.pview(), scale, o.pview(mut=True))) == eh.Status.OK, \
        eh.last_error()
    want = np.zeros_like(x)
    assert orc.soft_max_ext(a.oview(), m.oview(), scale, orc.view(want, a.ne)) == orc.OK
    got = o.result()
    assert np.isnan(want.reshape(nh, nq, nkv)[:, 0]).all()  # fully masked rows are NaN
    assert_close_rel(got, want, RTOL, "soft_max_ext fully masked / non-finite")
    assert (np.isnan(got) == np.isnan(want)).all()


# (4096, 2040) and (2048, 1592): the special rows among enough plain rows for one wave per row
@pytest.mark.parametrize("cols,extra", [(4096, 0), (256, 0), (20000, 0), (37, 0), (4096, 2040), (2048, 1592)])
def test_rms_norm_non_finite(gpu, cols, extra):
    # x*x overflows f32 (sum +inf, scale 0: finite x -> 0, inf x -> NaN), NaN
    # and inf elements, an all-zero row (scale 1/sqrt(eps)), subnormals
    g = np.random.Generator(np.random.PCG64(421 + cols))
    rows = []
    def base():
        return g.standard_normal(cols).astype(np.float32)
    r = base(); r[cols // 2] = np.float32(1e20); rows.append(r)
    r = base(); r[0] = np.inf; rows.append(r)
    r = base(); r[-1] = -np.inf; rows.append(r)
    r = base(); r[cols // 3] = np.nan; rows.append(r)
    rows.append(np.zeros(cols, np.float32))
    rows.append(np.full(cols, np.float32(1e-40)))
    r = base(); r[:] = np.float32(3e38); rows.append(r)
    rows.append(base())
    rows.extend(base() for _ in range(extra))
    x = np.concatenate(rows)
    n = len(rows)
    for ev, fn, what in ((lambda v, o: eh.OpRmsNorm(v, o, 1e-5), lambda a, o: orc.rms_norm(a, o, 1e-5), "rms_norm"),
                         (lambda v, o: eh.OpNorm(v, o, 1e-5), lambda a, o: orc.norm(a, o, 1e-5), "norm")):
        a = Pair(x, [cols, n, 1, 1]).to(gpu)
        o = Pair(np.zeros_like(x), a.ne).to(gpu)
        assert eh.Kernel().process_event(ev(a.pview(), o.pview(mut=True))) == eh.Status.OK, eh.last_error()
        want = np.zeros_like(x)
        assert fn(a.oview(), orc.view(want, a.ne)) == orc.OK
        got = o.result()
        assert_close_rel(got, want, RTOL, f"{what} non-finite, {cols} columns", atol=1e-30)
        assert (np.isnan(got) == np.isnan(want)).all(), what
