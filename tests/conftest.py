import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (run with -m gpu on the GPU box)")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Device for GPU tests.  Skips only when there is no GPU at all; on a GPU box
    a missing native library is an error, never a skip."""
    if not _gpu_available():
        pytest.skip("no GPU in this environment")
    import torch
    from qvggt_amd import _lib
    _lib.load()  # raises if libqvggt_hip.so is missing
    return torch.device("cuda:0")


def pytest_runtest_setup(item):
    # print which GPU case runs before it runs (so a box that dies names it)
    if "gpu" in item.keywords and os.environ.get("QVGGT_ECHO_TESTS", "1") == "1":
        print(f"\n[gpu-test] {item.nodeid}", flush=True)
