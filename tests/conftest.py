"""Shared pytest configuration: the `gpu` marker and import paths."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / 'gpu-libero_amd'):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (ROCm GPU) and the built libmx_physics.so')


@pytest.fixture(scope='session')
def gpu_available():
    import torch
    if not torch.cuda.is_available():
        pytest.skip('no ROCm GPU visible')
    return True
