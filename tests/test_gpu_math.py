"""GPU: exhaustive checks of the device shortcuts the kernels take, run on
the GPU itself (tests/native/gpu_checks.hip):

  hardware f32 -> f16 conversion == the reference's fp32_to_fp16 (all 2^32)
  hardware f16 -> f32 widening   == the reference's fp16_to_f32 (all 65536)
  emel_expf_nonpos              == emel_expf for every x <= 0 and NaN
  __builtin_sqrtf               correctly rounded for every input (power.rs)
"""
import ctypes
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "native" / "libgpu_checks.so"


@pytest.fixture(scope="module")
def checks(gpu):
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    L = ctypes.CDLL(str(LIB))
    for n in ("gpu_check_fp32_to_fp16", "gpu_check_fp16_to_f32", "gpu_check_expf_nonpos", "gpu_check_sqrtf"):
        getattr(L, n).restype = ctypes.c_uint64
        getattr(L, n).argtypes = []
    return L


@pytest.mark.parametrize("name", ["gpu_check_fp32_to_fp16", "gpu_check_fp16_to_f32", "gpu_check_expf_nonpos",
                                  "gpu_check_sqrtf"])
def test_exhaustive_on_gpu(checks, name):
    assert getattr(checks, name)() == 0
