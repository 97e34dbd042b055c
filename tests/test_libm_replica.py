"""CPU: the product's device math (emel.rs_amd/csrc/libm_replica.hpp), built
for the host by tests/native/libm_replica_check.cpp, against independent
checkers over ALL 2^32 float inputs:

  expf, expm1f, tanhf, logf, sinf, cosf, log1pf
                       == the host glibc (Rust std's f32::exp/exp_m1/tanh/ln/
                          sin/cos/ln_1p on x86_64-linux-gnu, i.e. what the
                          reference computes);
  fp32 -> fp16         == IEEE round-to-nearest-even (_Float16 conversion);
  fp16 -> fp32         == exact widening;
  GELU by polynomial and table
                       == the formula (the kernels' polynomial limits,
                          saturation thresholds and compact table layout);
  silu                 == x / (1 + glibc expf(-x)) (the kernels clamp
                          expf's argument instead of selecting its special
                          cases).

The GPU kernels run this same code, so a GPU result can differ from the
oracle only through the GPU's IEEE basic operations, which the GPU tests
check separately.
"""
import ctypes
import os
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parent / "native" / "libm_replica_check.so"
THREADS = max(1, min(8, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def chk():
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    L = ctypes.CDLL(str(LIB))
    for n in ("check_expf", "check_expm1f", "check_tanhf", "check_logf", "check_sinf", "check_cosf", "check_log1pf",
              "check_fp32_to_fp16", "check_gelu_table", "check_silu"):
        getattr(L, n).restype = ctypes.c_uint64
        getattr(L, n).argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int]
    L.check_fp16_to_f32.restype = ctypes.c_uint64
    for n in ("replica_silu", "replica_gelu", "replica_expf", "replica_tanhf"):
        getattr(L, n).restype = ctypes.c_float
        getattr(L, n).argtypes = [ctypes.c_float]
    return L


@pytest.mark.parametrize("fn", ["check_expf", "check_expm1f", "check_tanhf", "check_logf", "check_sinf", "check_cosf",
                                "check_log1pf", "check_fp32_to_fp16", "check_gelu_table", "check_silu"])
def test_exhaustive(chk, fn):
    assert getattr(chk, fn)(0, 1 << 32, THREADS) == 0


@pytest.mark.parametrize("negative", [0, 1])
def test_gelu_polynomial_range_is_maximal(chk, negative):
    """The kernels compute GELU by polynomial below an fp16 magnitude limit
    per sign and look the rest up; the exhaustive table check shows the
    polynomial right below each limit, this shows it fails at the limit, so
    the table holds exactly the values the polynomial cannot give."""
    chk.gelu_poly_first_miss.restype = ctypes.c_uint32
    chk.gelu_poly_first_miss.argtypes = [ctypes.c_int]
    chk.gelu_poly_limit.restype = ctypes.c_uint32
    chk.gelu_poly_limit.argtypes = [ctypes.c_int]
    limit = chk.gelu_poly_limit(negative)
    assert chk.gelu_poly_first_miss(negative) == limit
    assert limit == (0x34d0 if negative else 0x342e)


def test_fp16_widening(chk):
    assert chk.check_fp16_to_f32() == 0


def test_division_by_reciprocal_is_correctly_rounded(chk):
    """soft_max divides a row by its sum b >= 1 as RN24(RN53(a * RN53(1/b)));
    this must equal IEEE RN24(a / b).  Every a in [0, 1] (all the values a
    soft_max numerator takes) for divisors chosen to stress the argument
    (powers of two, all-ones significands, values near 1 and 2^k, random),
    plus random (a, b) pairs over the whole f32 line."""
    import numpy as np

    chk.check_div_recip.restype = ctypes.c_uint64
    chk.check_div_recip.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64,
                                     ctypes.c_int]
    chk.check_div_recip_random.restype = ctypes.c_uint64
    chk.check_div_recip_random.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int]
    g = np.random.Generator(np.random.PCG64(77))
    bs = np.array([1.0, 3.0, np.float32(2.0) - np.float32(2.0 ** -23), 1.0 + 2.0 ** -23, 4095.999755859375,
                   np.nextafter(np.float32(1024), np.float32(0))] + list(g.uniform(1, 4096, 2)), dtype=np.float32)
    one = int(np.float32(1.0).view(np.uint32))
    assert chk.check_div_recip(bs.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(bs), 0, one + 1, THREADS) == 0
    assert chk.check_div_recip_random(12345, 200_000_000, THREADS) == 0


def test_replica_matches_oracle_scalars(chk):
    import numpy as np

    import oracle as orc

    xs = np.concatenate([np.linspace(-12, 12, 20001, dtype=np.float32),
                         np.array([-10.1, -10.0, -1.2345, -0.125, 0.0, 0.12345, 10.0, 10.1], np.float32)])
    for x in xs:
        x = float(x)
        assert np.float32(chk.replica_silu(x)).view(np.uint32) == np.float32(orc.silu_scalar(x)).view(np.uint32), x
        assert np.float32(chk.replica_gelu(x)).view(np.uint32) == np.float32(orc.gelu_scalar(x)).view(np.uint32), x


def test_exact_sequential_sum_rounds(chk):
    """The sampler's exact sequential f32 sum (seqsum.hpp; sampler.hip's
    k_smp_seg and k_smp_sum) emulated on the host: integer units per binade,
    ties, binade crossings, NaN and +inf taken as single f32 additions, and
    chunk contributions predicted from f64 chunk sums and taken only when
    the exact state confirms them.  It must give the bits of a plain
    sequential f32 loop.  Families: softmax-like values, dyadic values full
    of exact ties, zeros and subnormals, every magnitude, planted NaN / +inf;
    the walk alone (64 lanes, as the kernel, and 4) and with predictions
    (config 5's 5120-element chunks of 512-element sub-chunks as the kernel
    walks them, 4748-element chunks, 100- and 1024-element chunks).  Ignoring ties, or
    letting a binade run to 2^25 units, makes this check fail."""
    chk.check_seqsum.restype = ctypes.c_uint64
    chk.check_seqsum.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_uint64]
    assert chk.check_seqsum(1, 2000, 300) == 0
    assert chk.check_seqsum(2, 40, 200_000) == 0


def test_exact_sum_from_approximate_prefixes(chk):
    """The fused path (sampler.hip's k_smp_max<true> + k_smp_expseg) predicts
    from approximate sums, with the bounds widened by 2^-14.  Correctness
    rests on the walk's checks alone: prefixes perturbed within that margin,
    and far beyond it (1%; 50%, which steers many predictions to a wrong
    binade), must still give the bits of the sequential loop.  On a
    config-5-like row the small perturbations take as many sub-chunks in one
    step as exact prefixes do (a sub-chunk whose bounds span two binades is
    counted at both), and the large one fewer."""
    import numpy as np

    chk.check_seqsum_approx.restype = ctypes.c_uint64
    chk.check_seqsum_approx.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_uint64, ctypes.c_double,
                                        ctypes.c_double]
    assert chk.check_seqsum_approx(3, 1000, 20_000, 2.0**-16, 2.0**-14) == 0
    assert chk.check_seqsum_approx(4, 1000, 20_000, 1e-2, 2.0**-14) == 0
    assert chk.check_seqsum_approx(5, 1000, 20_000, 0.5, 0.0) == 0
    chk.seqsum_approx_f.restype = ctypes.c_float
    chk.seqsum_approx_f.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64,
                                    ctypes.c_uint64, ctypes.c_double, ctypes.c_double, ctypes.c_uint64,
                                    ctypes.POINTER(ctypes.c_uint64)]
    g = np.random.Generator(np.random.PCG64(6))
    v = (g.standard_normal(151936) / 0.8).astype(np.float32)
    e = np.exp((v - v.max()).astype(np.float64)).astype(np.float32)
    want = np.cumsum(e, dtype=np.float32)[-1]
    ptr = e.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    taken = {}
    for perturb, widen in ((0.0, 0.0), (2.0**-16, 2.0**-14), (1e-2, 2.0**-14), (0.5, 0.0)):
        jumped = ctypes.c_uint64(0)
        got = chk.seqsum_approx_f(ptr, e.size, 32, 5120, 512, perturb, widen, 7, ctypes.byref(jumped))
        assert np.float32(got) == want, perturb
        taken[perturb] = jumped.value
    assert taken[2.0**-16] >= taken[0.0] - 2, taken
    assert taken[1e-2] >= taken[0.0] - 2, taken
    assert taken[0.5] < taken[0.0], taken


def test_exact_sum_predictions_are_taken(chk):
    """On a config-5-like row (softmax of N(0,1) logits / 0.8 over 151,936
    tokens) most sub-chunks are taken from their prediction in one step: the
    walk is left with the sub-chunks where the binade changes.  Sub-chunks
    whose bounds span two binades are counted at both, so only the ones that
    cross are walked: 288 of 297 at 512 elements, where a count at one binade
    took 285."""
    import numpy as np

    chk.seqsum_chunked_f.restype = ctypes.c_float
    chk.seqsum_chunked_f.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_uint64, ctypes.c_uint32,
                                     ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]
    g = np.random.Generator(np.random.PCG64(5))
    v = (g.standard_normal(151936) / 0.8).astype(np.float32)
    e = np.exp((v - v.max()).astype(np.float64)).astype(np.float32)
    want = np.cumsum(e, dtype=np.float32)[-1]
    # the kernel's shape: 5120-element chunks of 512-element sub-chunks
    # (297 of them), and 4748-element chunks of 1024-element ones (160)
    for lanes, chunk, sub, least in ((32, 5120, 512, 287), (64, 4748, 1024, 150)):
        jumped = ctypes.c_uint64(0)
        got = chk.seqsum_chunked_f(e.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), e.size, lanes, chunk, sub,
                                   ctypes.byref(jumped))
        assert np.float32(got) == want
        assert jumped.value >= least, (sub, jumped.value)
