"""Shared test setup.

Markers: ``gpu`` tests need a real MI355X and call the kernels through the C
ABI (``braid_amd.kernels.loader``); everything else runs on the CPU.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
HERE = Path(__file__).resolve().parent
if str(HERE) not in sys.path:
    sys.path.insert(0, str(HERE))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def kern():
    """The loaded kernel module. GPU tests only."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from braid_amd.kernels.loader import load_gdn

    return load_gdn()
