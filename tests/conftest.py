"""Shared test setup: the `gpu` marker, loading the product package (its
directory name holds a hyphen, so it is loaded by path) and the oracle."""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_pkg():
    name = "bark3_wgpu_amd"
    if name in sys.modules:
        return sys.modules[name]
    # torch ships its own HIP runtime under the same soname as ROCm's. Whichever
    # loads first serves the process; torch only finds the GPU on its own copy,
    # so it is imported before the library pulls in ROCm's.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    init = ROOT / "bark3-wgpu_amd" / "__init__.py"
    spec = importlib.util.spec_from_file_location(name, init, submodule_search_locations=[str(init.parent)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def synth(pkg):
    import importlib

    return importlib.import_module("bark3_wgpu_amd.synth")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


def rel_max_abs(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want| — the per-block tolerance metric."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))
