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


# ------------------------------------------------------------------ parity margins on record
# Tests hand each measured error and its bound to the `parity` fixture; with DIFFLET_PARITY_LOG
# set, the session writes them (test, quantity, error, bound, bound / error) as a markdown
# table to that path, so the margin under every tolerance is kept, not only pass / fail.
_PARITY: list = []


@pytest.fixture
def parity(request):
    def record(quantity: str, value: float, bound: float) -> None:
        _PARITY.append((request.node.nodeid, quantity, float(value), float(bound)))

    return record


# Long GPU tests (the full-depth steps against the host oracle, minutes of CPU work) report
# their progress through `progress`, which writes past pytest's output capture, so a quiet
# (-q) run still shows them advancing.
@pytest.fixture
def progress(request):
    capman = request.config.pluginmanager.getplugin("capturemanager")

    def emit(msg: str) -> None:
        if capman is None:
            print(msg, flush=True)
            return
        with capman.global_and_fixture_disabled():
            print(msg, flush=True)

    return emit


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("DIFFLET_PARITY_LOG")
    if not path or not _PARITY:
        return
    lines = ["| test | quantity | measured | bound | bound / measured |",
             "|---|---|---:|---:|---:|"]
    for node, q, v, b in _PARITY:
        ratio = f"{b / v:.1f}" if v > 0 else "inf"
        lines.append(f"| `{node}` | {q} | {v:.3e} | {b:.1e} | {ratio} |")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
