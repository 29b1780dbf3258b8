"""Shared test fixtures.

Markers: `gpu` — needs the MI355X (run with `-m gpu` on the GPU machine);
everything else runs on the CPU-only build container.
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)

PKG_DIR = os.path.join(ROOT, "cuda-msst-infer_amd")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP kernels)")


def load_msst():
    """Import the package directory (its name has dashes) as `msst_amd`."""
    if "msst_amd" in sys.modules:
        return sys.modules["msst_amd"]
    spec = importlib.util.spec_from_file_location(
        "msst_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["msst_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def msst():
    return load_msst()


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch.device("cuda:0")


def rel_err(y, r) -> float:
    """Normwise relative error max|y - r| / max|r| (the parity metric)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    assert y.shape == r.shape, (y.shape, r.shape)
    assert np.all(np.isfinite(y)), "non-finite values in result"
    denom = np.max(np.abs(r))
    if denom == 0.0:
        return float(np.max(np.abs(y)))
    return float(np.max(np.abs(y - r)) / denom)


def elem_rel_err(y, r, floor_frac=1e-3) -> float:
    """Element-wise relative error with a floor of floor_frac * max|r|."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    floor = floor_frac * np.max(np.abs(r))
    return float(np.max(np.abs(y - r) / np.maximum(np.abs(r), floor)))


TOL_F32 = 1e-4   # fp32 path: max relative error (normwise)
TOL_F16 = 2e-2   # fp16 path (fp16 outputs, fp32 accumulation)
