"""GPU: the plain-C caller (tests/native/c_caller.c, built by
__graft_entry__.build()) drives the C ABI on device 0 with no Python in
the loop: library-allocated device buffers, broadcast add, scaled + masked
soft_max, per-row argmax, the logits validator and the sampler (after
reserving the stream's scratch and building the device tables), each
checked inside the program."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "native" / "c_caller"


def test_c_caller_on_the_gpu():
    if not EXE.exists():
        pytest.fail("tests/native/c_caller is not built: run __graft_entry__.build()")
    print("c_caller gpu", flush=True)
    r = subprocess.run([str(EXE), "gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "c_caller gpu: ok" in r.stdout, r.stdout + r.stderr
