"""pytest setup: the `gpu` marker, and the built libraries.

`-m "not gpu"` runs everything that needs no GPU (oracle pins, host logic,
ABI checks); `-m gpu` runs the parity tests on the device. Libraries are built
only when missing; after changing a source, run __graft_entry__.build().
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

SEED = 20261005  # the reference test runner's default seed (tests/test_main.cpp:23)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP kernels)")


@pytest.fixture(scope="session", autouse=True)
def _built_libraries():
    import oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    from ember_amd import build as b

    if not b.LIB.exists():
        b.build()
    driver = ROOT / "tests" / "cpp" / "_build" / "hip_engine_test"
    if not driver.exists():
        import importlib.util

        spec = importlib.util.spec_from_file_location("cpp_drivers", ROOT / "tests" / "cpp" / "build.py")
        drivers = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(drivers)
        drivers.build()
    yield


@pytest.fixture
def rng():
    import numpy as np

    return np.random.default_rng(SEED)


@pytest.fixture(scope="session")
def device():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")
