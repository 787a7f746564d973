"""pytest configuration: the `gpu` marker and shared fixtures.

Tests marked `gpu` need a visible MI355X and call the HIP library through its
C-ABI; the rest run on any host (no compute calls without a GPU).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

# torch bundles its own HIP runtime; libf3s_hip.so binds to whichever
# libamdhip64.so.7 the process loads first.  Importing torch before any test
# touches the library keeps one runtime in the test process, so the torch
# binding's tests can share it with the rest of the suite.
try:
    import torch  # noqa: F401
except ImportError:   # the library itself does not need torch
    torch = None

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X, gfx950) and runs HIP kernels")
    config.addinivalue_line("markers", "slow: large configuration (seconds to minutes)")


@pytest.fixture(scope="session")
def gpu():
    """Fails (not skips) if no device: the GPU suite must run the HIP path."""
    import fused3s_amd as f3s
    n = f3s.device_count()
    assert n >= 1, "no HIP device visible: the gpu tests need an MI355X"
    return f3s


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def random_csr(n: int, avg_deg: float, seed: int, self_loops: bool = True, sym: bool = True):
    """Small random simple graph as CSR (sorted unique columns)."""
    r = rng(seed)
    m = int(n * avg_deg / 2)
    u = r.integers(0, n, m)
    v = r.integers(0, n, m)
    keep = u != v
    u, v = u[keep], v[keep]
    if sym:
        u, v = np.concatenate([u, v]), np.concatenate([v, u])
    if self_loops:
        u = np.concatenate([u, np.arange(n)])
        v = np.concatenate([v, np.arange(n)])
    key = np.unique(u.astype(np.int64) * n + v)
    rows, cols = key // n, key % n
    row_ptr = np.zeros(n + 1, np.int64)
    np.add.at(row_ptr, rows + 1, 1)
    return np.cumsum(row_ptr).astype(np.int32), cols.astype(np.int32)
