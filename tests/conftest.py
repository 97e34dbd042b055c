import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "emel.rs_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libemel_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """The torch device for GPU tests; skips when no GPU is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import emel_hip

    emel_hip.load()  # raises if the HIP library is missing: no silent fallback
    if emel_hip.device_count() < 1:
        pytest.fail("a GPU is visible but it is not gfx950")
    return torch.device("cuda:0")
