"""GPU: exhaustive checks of the device shortcuts the kernels take, run on
the GPU itself (tests/native/gpu_checks.hip):

  hardware f32 -> f16 conversion == the reference's fp32_to_fp16 (all 2^32)
  hardware f16 -> f32 widening   == the reference's fp16_to_f32 (all 65536)
  emel_expf_nonpos              == emel_expf for every x <= 0 and NaN
  emel_silu (clamped expf argument) == x / (1 + emel_expf(-x)) (all 2^32)
  GELU by polynomial and table  == emel_gelu (all 2^32), with the hardware
                                fp16 conversions the kernels use
  __builtin_sqrtf               correctly rounded for every input (power.rs)
  f64 sqrt and division         IEEE results on 2^23 random doubles (the generic
                                norms' f64 scale), compared with numpy on the host
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "native" / "libgpu_checks.so"


@pytest.fixture(scope="module")
def checks(gpu):
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    L = ctypes.CDLL(str(LIB))
    for n in ("gpu_check_fp32_to_fp16", "gpu_check_fp16_to_f32", "gpu_check_expf_nonpos", "gpu_check_sqrtf",
              "gpu_check_silu", "gpu_check_gelu"):
        getattr(L, n).restype = ctypes.c_uint64
        getattr(L, n).argtypes = []
    return L


@pytest.mark.parametrize("name", ["gpu_check_fp32_to_fp16", "gpu_check_fp16_to_f32", "gpu_check_expf_nonpos",
                                  "gpu_check_sqrtf", "gpu_check_silu", "gpu_check_gelu"])
def test_exhaustive_on_gpu(checks, name):
    assert getattr(checks, name)() == 0


def test_f64_sqrt_and_division_are_ieee(checks):
    g = np.random.Generator(np.random.PCG64(64))
    n = 1 << 23
    x = g.integers(0, 1 << 63, n, dtype=np.uint64).view(np.float64).copy()  # positive, every exponent
    y = g.integers(0, 1 << 64, n, dtype=np.uint64, endpoint=False).view(np.float64).copy()
    x[:8] = [0.0, -0.0, np.inf, 1.0, 2.0, 5e-324, 1.7976931348623157e308, 0.25]
    sq = np.empty_like(x)
    dv = np.empty_like(x)
    P = ctypes.POINTER(ctypes.c_double)
    checks.gpu_f64_ops.restype = ctypes.c_uint64
    checks.gpu_f64_ops.argtypes = [P, P, P, P, ctypes.c_uint64]
    assert checks.gpu_f64_ops(x.ctypes.data_as(P), y.ctypes.data_as(P), sq.ctypes.data_as(P),
                              dv.ctypes.data_as(P), n) == 0
    with np.errstate(all="ignore"):
        want_sq = np.sqrt(x)
        want_dv = x / y
    for got, want, what in ((sq, want_sq, "sqrt"), (dv, want_dv, "division")):
        same = (got.view(np.uint64) == want.view(np.uint64)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (what, int((~same).sum()), x[~same][:4], got[~same][:4], want[~same][:4])
