import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an AMD Instinct GPU and the built libredshift_hip')


@pytest.fixture(scope='session')
def lib():
    """The in-tree libredshift_hip (a missing build is an error, not a skip)."""
    from redshift_amd.runtime import load_library
    return load_library()


@pytest.fixture(scope='session')
def gpu():
    """Skip when no GPU is visible; otherwise return the torch module."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip('no GPU visible')
    return torch
