"""Test configuration: markers, import paths and shared fixtures.

`-m "not gpu"` runs the oracle pins, host logic and ABI checks on the CPU;
`-m gpu` runs the parity tests through the C-ABI on a real MI355X.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("pop2-bezier_amd", "oracle", "tests"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X; run the CPU suite with -m 'not gpu'")
    return torch.device("cuda:0")
