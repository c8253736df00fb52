"""Shared pytest setup.

`-m "not gpu"` runs here without a GPU: oracle pinning, host logic (C++
unit tests), and C-ABI load/export checks.  `-m gpu` tests are the parity
tests proper: they call the HIP library through the C ABI (ctypes) and
compare with the CPU oracle.
"""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tensor-ash_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ta():
    import tensor_ash
    return tensor_ash


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    return o


@pytest.fixture(scope="session")
def ctx(ta):
    return ta.Context()


@pytest.fixture(scope="session")
def ex(ta, ctx):
    # tune=False keeps routing on the static heuristic (tests/common/mod.rs:23-29)
    return ta.Executor(ctx, n_slots=2, max_calls_per_submit=64, tune=False)


def rel_err(got, ref) -> float:
    """Normwise relative error: max |got - ref| / max |ref|."""
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    ref = np.asarray(ref, dtype=np.float64).reshape(-1)
    if not np.all(np.isfinite(got)):
        return float("inf")
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))
