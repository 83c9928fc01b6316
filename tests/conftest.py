"""Shared fixtures.  `gpu`-marked tests run on an MI355X and call the HIP path
through the C-ABI; everything else runs on the CPU (oracle pinning, golden
fixtures, host logic, library exports)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _have_gpu() -> bool:
    try:
        from final_amd import hip
        return hip.device_count() > 0
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if any("gpu" in item.keywords for item in items) and not _have_gpu():
        skip = pytest.mark.skip(reason="no HIP device visible")
        for item in items:
            if "gpu" in item.keywords:
                item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def real_weights():
    """Seed-0 weights at the reference shapes (1.41 GB, generated once)."""
    from final_amd import workloads as W
    return W.gen_weights(0)


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
