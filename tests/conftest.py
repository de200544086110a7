import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    config.addinivalue_line("markers", "slow: long-running CPU oracle work")


@pytest.fixture(scope="session")
def dev():
    """The HIP device; GPU tests fail (not skip) when none is present, as the
    reference's CUDA tests do (crates/tang-compute/src/cuda.rs:4195)."""
    from tang_amd import capi
    assert capi.device_count() > 0, "no HIP GPU visible"
    d = capi.HipComputeDevice(0)
    yield d
    d.close()


def max_abs_rel(got, ref):
    """max |got - ref| / max |ref| (the tolerance metric of the parity tests)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = max(np.max(np.abs(ref)), 1e-30)
    return float(np.max(np.abs(got - ref)) / denom)
