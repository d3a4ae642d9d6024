import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The device for gpu-marked tests; the library must be built and load (no fallback)."""
    if not _gpu_available():
        pytest.skip("no GPU on this host")
    import torch

    from difflet_amd import _lib

    _lib.load()
    return torch.device("cuda", 0)
