"""pytest configuration: the ``gpu`` marker and shared helpers.

``-m "not gpu"`` runs the oracle, host-logic and ABI-export tests (no GPU);
``-m gpu`` runs the parity tests, which call the HIP kernels through the C ABI.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libfk_amd.so")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from fastkernels_amd import _native

    _native.lib()  # fail loudly if the library is missing
    return torch.device("cuda:0")
