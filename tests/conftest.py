"""Shared pytest setup.

Tests marked ``gpu`` need an MI355X and the built libkvpath.so; everything else runs
on the CPU.  The repository root is put on sys.path so ``oracle`` and ``kavor_amd``
import without installation.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and libkvpath.so")


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a GPU test was selected but no GPU is visible")
    from kavor_amd._lib import lib

    lib()  # fail loudly if the HIP library is missing
    return torch.device("cuda", 0)
