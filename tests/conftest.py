"""Shared test setup: put the package on sys.path, register the ``gpu`` marker,
and provide small helpers (CPU-seeded inputs, cosine / max-abs metrics)."""

from __future__ import annotations

import os
import sys

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "low-bit-attention-fake-quant_amd")
for p in (REPO, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def cpu_randn(*shape, seed=0, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def cosine(a, b):
    """Cosine similarity in float64 (a float32 reduction over ~10^6 elements is
    off by ~10^-5)."""
    a = a.double().flatten()
    b = b.double().flatten()
    return ((a @ b) / (a.norm() * b.norm()).clamp_min(1e-300)).item()


def max_abs(a, b):
    return (a.float() - b.float()).abs().max().item()


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from low_bit_fake_quant import _lib
    _lib.load()
    return torch.device("cuda:0")
