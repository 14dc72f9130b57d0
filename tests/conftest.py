import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0; GPU tests fail (never skip) without it."""
    import torch

    from warpgbm_amd import _lib

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    lib = _lib.load()
    return lib


def c1_data(n=10000, f=50, seed=0):
    """Config C1: X ~ N(0,1) float32, y = X.w (10 nonzero) + 0.1 N(0,1), 10k x 50."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, f), dtype=np.float32)
    w = np.zeros(f, np.float32)
    idx = rng.choice(f, 10, replace=False)
    w[idx] = rng.standard_normal(10)
    y = (X @ w + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return X, y


def print_case(*parts):
    """Name the case before a GPU step (flushed, so it survives a lost box)."""
    print("CASE:", *parts, flush=True)
