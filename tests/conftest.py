"""Test configuration: the `gpu` marker, import paths and shared helpers.

CPU tests (`-m "not gpu"`) check the oracle against the golden vectors and the
mathematics, the host code (quantizer, registry, argument checks) and that
libtiermm.so exports every symbol include/tiermm.h declares.  GPU tests
(`-m gpu`) call the HIP kernels through the C ABI and compare with the oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtiermm.so")


def _has_gpu() -> bool:
    try:
        from tier_amd import hip
        return hip.device_count() > 0
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if any("gpu" in item.keywords for item in items) and not _has_gpu():
        skip = pytest.mark.skip(reason="no HIP device visible")
        for item in items:
            if "gpu" in item.keywords:
                item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    g = os.path.join(TESTS, "golden")
    return {
        "dequant": np.load(os.path.join(g, "dequant_golden.npz")),
        "quant": np.load(os.path.join(g, "quant_golden.npz")),
        "f16": np.load(os.path.join(g, "f16_golden.npz")),
    }


@pytest.fixture(scope="session")
def gpu():
    """Initialise the library on device 0 once per session."""
    import tier_amd
    from tier_amd import hip
    hip.set_device(0)
    tier_amd.init(0)
    yield tier_amd
    hip.synchronize()
