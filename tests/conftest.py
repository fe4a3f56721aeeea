"""Pytest configuration: the ``gpu`` marker and shared fixtures.

Tests marked ``gpu`` need an MI355X (gfx950) and the built HIP extension;
everything else runs on the CPU.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP extension")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from akas_amd import _lib

    _lib.load()  # fails loudly when the extension is missing
    return torch.device("cuda:0")
