import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

KERNEL_SEED = 20260819  # reference validate_kernels.py:122
MODEL_SEED = 20260625   # reference benchmark_public.py:72


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libq35.so)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def gpu():
    import torch

    assert torch.cuda.is_available(), "GPU tests need an MI355X; none is visible"
    from ppu_amd import _lib

    _lib.load()
    return torch.device("cuda:0")


def gen(seed: int):
    import torch

    return torch.Generator().manual_seed(seed)
