import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests never fall back: without a GPU they fail, not skip."""
    if not _gpu_available():
        pytest.fail("no GPU visible: the -m gpu tests need an MI355X")
    import torch
    from neuroflow_amd import _lib
    _lib.lib()   # raises if libnflow_quant.so is not built
    return torch.device("cuda:0")
