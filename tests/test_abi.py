"""CPU: the C-ABI library loads, exports every symbol include/emel_hip.h
declares, and its host-side guards agree with the oracle's restatement of
the reference's view rules.  No kernel is launched."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import emel_hip as eh
import oracle as orc
from emel_hip.abi import CView

HEADER = Path(__file__).resolve().parents[1] / "include" / "emel_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(emel_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = eh.load()
    names = declared_functions()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_and_status_strings():
    lib = eh.load()
    assert lib.emel_abi_version() == 2
    for s in eh.Status:
        assert lib.emel_status_string(int(s)).decode()


def test_struct_layout_matches_header():
    # emel_tensor_view: pointer, u32 dtype, u32 reserved, u64[4], u64[4], u64 data_bytes -- the pinned
    # C++ tensor_view {data, type, ne, nb} (80 bytes) followed by data_bytes
    assert ctypes.sizeof(CView) == 8 + 4 + 4 + 32 + 32 + 8
    assert CView.dtype.offset == 8 and CView.ne.offset == 16 and CView.nb.offset == 48
    assert CView.data_bytes.offset == 80


def random_layouts(seed, count):
    g = np.random.Generator(np.random.PCG64(seed))
    for _ in range(count):
        ne = [int(g.integers(0, 5)) if g.random() < 0.1 else int(g.integers(1, 6)) for _ in range(4)]
        mode = g.integers(0, 4)
        if mode == 0:
            nb = [0, 0, 0, 0]
        elif mode == 1:
            nb = [4]
            for d in range(1, 4):
                nb.append(nb[-1] * ne[d - 1])
        else:
            nb = [int(g.choice([0, 2, 4, 6, 8, 12, 16, 20, 64, 100, 400])) for _ in range(4)]
        dtype = int(g.choice([0, 0, 0, 0, 1, 26]))
        data_bytes = int(g.integers(0, 2000))
        yield ne, nb, dtype, data_bytes


def cview(ne, nb, dtype, data_bytes, ptr=0x1000):
    v = CView()
    v.data = ptr
    v.data_bytes = data_bytes
    v.dtype = dtype
    v.reserved = 0
    for d in range(4):
        v.ne[d] = ne[d]
        v.nb[d] = nb[d]
    return v


def test_host_view_guards_match_oracle():
    lib = eh.load()
    backing = np.zeros(1, np.float32)
    for ne, nb, dtype, nbytes in random_layouts(5, 20000):
        ov = orc.view(backing, ne, nb, dtype, nbytes)
        v = cview(ne, nb, dtype, nbytes)
        for allow in (0, 1):
            want = orc.call("orc_layout_validate", ov, allow) == orc.OK
            got = lib.emel_validate_view(ctypes.byref(v), allow) == 0
            assert got == want, (ne, nb, dtype, nbytes, allow)
        want = orc.call("orc_normalization_view_valid", ov) == 1
        got = lib.emel_validate_normalization_view(ctypes.byref(v)) == 0
        assert got == want, (ne, nb, dtype, nbytes, "normalization")


def _no_gpu():
    return eh.device_count() == 0


@pytest.mark.skipif(not _no_gpu(), reason="host-pointer rejection checks only run where no GPU is visible")
def test_rejections_run_on_the_host_before_any_device_work():
    """Invalid requests are classified on the host, exactly as the reference's
    guards classify them, and the host buffers stay untouched."""
    a = np.ones(4, np.float32)
    o = np.full(3, 9.0, np.float32)

    def hv(arr, ne, nb=None, dtype=0, nbytes=None):
        nb = nb or [4, 4 * ne[0], 4 * ne[0] * ne[1], 4 * ne[0] * ne[1] * ne[2]]
        return cview(ne, nb, dtype, arr.nbytes if nbytes is None else nbytes, arr.ctypes.data)

    lib = eh.load()
    r = ctypes.byref
    A = hv(a, [4, 1, 1, 1])
    O = hv(o, [3, 1, 1, 1])
    assert lib.emel_op_add(r(A), r(A), r(O), None) == eh.Status.SHAPE_MISMATCH
    assert lib.emel_op_unary(10, r(A), r(O), None) == eh.Status.UNEXPECTED_EVENT
    assert lib.emel_op_silu(r(A), r(O), None) == eh.Status.SHAPE_MISMATCH
    bad = hv(a, [4, 1, 1, 1], nbytes=12)
    assert lib.emel_op_mul(r(bad), r(A), r(A), None) == eh.Status.INVALID_VIEW
    A6 = hv(np.ones(6, np.float32), [3, 2, 1, 1])
    assert lib.emel_op_rms_norm(r(A6), r(A6), ctypes.c_float(float("nan")), None) == eh.Status.INVALID_PARAMETERS
    assert lib.emel_op_soft_max(r(A6), r(O), None) == eh.Status.SHAPE_MISMATCH
    assert lib.emel_op_sum_rows(r(A6), r(O), None) == eh.Status.SHAPE_MISMATCH
    assert (o == 9.0).all() and (a == 1.0).all()
    # an accepted request needs the device: no CPU fallback
    A3 = hv(np.ones(3, np.float32), [3, 1, 1, 1])
    assert lib.emel_op_add(r(A3), r(A3), r(O), None) == eh.Status.KERNEL_UNAVAILABLE
    assert (o == 9.0).all()


def test_plain_c_caller_compiles_links_and_runs(tmp_path):
    """include/emel_hip.h is valid strict C99 and a C program links the
    library with no C++ or Python around it (what a Rust, cgo or JNI binding
    does); on this host it runs the host-only entry points and sees the
    accepted op reported as KERNEL_UNAVAILABLE, never run on the CPU."""
    import subprocess

    import __graft_entry__ as ge

    if not (ge.PKG / "emel_hip" / "libemel_hip.so").exists():
        pytest.skip("libemel_hip.so is not built")
    exe = tmp_path / "c_caller"
    r = subprocess.run(ge.c_caller_command(exe, str(ge.PKG / "emel_hip")), capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    import torch

    mode = "gpu" if torch.cuda.is_available() else "cpu"
    r = subprocess.run([str(exe), mode], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and f"c_caller {mode}: ok" in r.stdout, r.stdout + r.stderr
