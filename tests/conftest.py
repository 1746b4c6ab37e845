"""Shared pytest setup: the `gpu` marker, import paths and tolerance helpers.

GPU tests call the HIP backend through its C ABI and compare against the CPU
oracle (oracle/, test infrastructure) or against committed fixtures.  They
never skip for a missing device: on a GPU box a missing device is a failure.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "vestra-kernels_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


@pytest.fixture(scope="session")
def rt():
    import vestra_hip

    return vestra_hip.Runtime(0)


def max_rel(actual, expected) -> float:
    """max |a - e| / max |e|: the normwise relative error the parity bars use."""
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    scale = np.abs(e).max() if e.size else 0.0
    if scale == 0.0:
        return float(np.abs(a - e).max()) if e.size else 0.0
    return float(np.abs(a - e).max() / scale)


def assert_bits_equal(actual, expected, what=""):
    a = np.ascontiguousarray(actual, np.float32).view(np.uint32)
    e = np.ascontiguousarray(expected, np.float32).view(np.uint32)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    bad = np.nonzero(a != e)[0]
    assert bad.size == 0, (
        f"{what}: {bad.size} of {a.size} values differ; first at {bad[0]}: "
        f"{np.float32(actual.reshape(-1)[bad[0]])} vs {np.float32(expected.reshape(-1)[bad[0]])}")
