import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Skip when no GPU is visible; on a GPU box the HIP library must be built."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from spmv_decode_amd import _lib

    _lib.load()  # raises if the library is missing: no silent fallback
    return torch.device("cuda:0")


def say(msg: str) -> None:
    """Progress line that names the case before GPU work (visible with -s)."""
    print(msg, flush=True)
