"""Shared pytest configuration.

Markers:
  gpu  -- needs a real MI355X (HIP device); the CPU suite runs with -m "not gpu".
"""

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs a GPU (HIP device) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.skip("GPU required")
    from triangleops_amd import _native

    _native.load()  # fail loudly (ImportError) if the HIP library is missing on a GPU box
    return torch.device("cuda:0")
