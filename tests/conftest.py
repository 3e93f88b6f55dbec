"""Shared test setup.

Markers: ``gpu`` -- needs a visible MI355X and calls libflock_attn through the C
ABI. Everything else runs on the CPU (oracle pinning, host logic, ABI exports).
"""
from __future__ import annotations

import os
import zlib
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (runs libflock_attn kernels)")


def _gpu_count() -> int:
    """Visible GPUs, counted without our library: with a GPU present a missing or
    broken libflock_attn.so must fail the gpu tests, not skip them."""
    try:
        import torch
        return torch.cuda.device_count()
    except Exception:
        return 0


def pytest_collection_modifyitems(config, items):
    if _gpu_count() > 0:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


# ------------------------------------------------------------------ helpers --
def randn(rng: np.random.Generator, n: int) -> np.ndarray:
    """N(0, 1) values as f32 (the benchmark workloads' inputs)."""
    return rng.standard_normal(n, dtype=np.float32)


def rand_unit(rng: np.random.Generator, n: int, scale: float = 1.0) -> np.ndarray:
    """Uniform [-scale, scale) as f32 -- the reference's randVec (lib.ts:595-599)."""
    return ((rng.random(n, dtype=np.float64) - 0.5) * 2 * scale).astype(np.float32)


@pytest.fixture
def rng(request):
    """A generator seeded from the test's id (stable across runs and machines)."""
    return np.random.default_rng(zlib.crc32(request.node.nodeid.encode()))
