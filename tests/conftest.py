import os
import sys
from pathlib import Path

import pytest

try:  # first import on a fresh box is slow: keep it out of per-test timeouts
    import torch  # noqa: F401
except Exception:  # pragma: no cover
    torch = None

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The device-side library, initialised; the test errors (not skips)
    when the HIP library is missing on a GPU box."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from logan_amd import backend

    assert backend.hip_init(), "logan-hip failed to initialise on this GPU"
    return torch.device("cuda:0")
