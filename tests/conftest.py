import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs the parity tests through the C-ABI")


@pytest.fixture(scope="session")
def gpu():
    """The CUDA/HIP device; GPU tests fail (never skip) without one."""
    import torch

    assert torch.cuda.is_available(), "gpu-marked test needs a HIP device"
    from loopspec_amd import _lib

    _lib.load()
    return torch.device("cuda", 0)


def announce(msg: str) -> None:
    """Flush a line naming the case before a GPU step, so a fault is attributable."""
    sys.__stdout__.write(f"[case] {msg}\n")
    sys.__stdout__.flush()
