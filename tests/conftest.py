"""Shared pytest setup: import paths, the `gpu` marker, and GPU availability."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "flash-attn-economical-gpu_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    """Skip (with the reason) when no GPU is visible; on the GPU box this always runs."""
    if not gpu_available():
        pytest.skip("no GPU visible (gfx950 required)")
    import torch

    return torch.device("cuda:0")
