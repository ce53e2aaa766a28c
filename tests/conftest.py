"""Shared pytest configuration.

``-m gpu`` tests run the HIP kernels on an MI355X and compare them with the CPU oracle
(oracle/) on identical seeded inputs; everything else runs on the CPU.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; GPU tests are skipped (not faked) when there is none."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU available")
    import cuda_transformer_amd  # noqa: F401  (fails loudly if the native library is missing)

    return torch.device("cuda", 0)


@pytest.fixture
def bwd_cap():
    """set_cap(nbytes) sets the flash_attention_bwd dS workspace cap for one test; the cap in force
    before the test is restored afterwards (the cap is process-wide)."""
    from cuda_transformer_amd import _C

    saved = []

    def set_cap(nbytes):
        prev = _C.set_bwd_workspace_cap(nbytes)
        if not saved:
            saved.append(prev)

    yield set_cap
    if saved:
        _C.set_bwd_workspace_cap(saved[0])


def seeded(shape, seed, kind="randn", scale=1.0):
    """float32 host tensor from a fixed CPU generator (identical bits for GPU and oracle)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    if kind == "randn":
        t = torch.randn(shape, generator=g, dtype=torch.float32)
    else:
        t = torch.rand(shape, generator=g, dtype=torch.float32)
    return t * scale if scale != 1.0 else t


def f64(t):
    return t.detach().cpu().double().numpy()


def rel_err(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_rel_err(a, b, tol=1e-3, floor=1e-6):
    """Relative L2 error <= tol (the acceptance bar for gradients).  When the reference is exactly zero
    up to rounding (norm below floor * sqrt(size), e.g. dQ for T = 1) a relative error is
    meaningless and the absolute bar floor * sqrt(size) applies instead."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    scale = floor * np.sqrt(b.size)
    if np.linalg.norm(b) <= scale:
        assert np.linalg.norm(a - b) <= scale
    else:
        assert rel_err(a, b) <= tol
