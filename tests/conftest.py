"""Test configuration: import paths, the ``gpu`` marker and shared helpers.

``-m "not gpu"`` runs the oracle, host-logic and ABI-surface tests on any
machine.  ``-m gpu`` runs the parity tests through libw8a8_gfx950.so on a
GPU; they skip only when no GPU is visible, and fail (never fall back) when
the library is missing.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "nano-pointllm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and libw8a8_gfx950.so")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from nanopointllm_amd import _lib

    _lib.load()  # raises if the HIP library is missing: no silent fallback
    return torch.device("cuda:0")
