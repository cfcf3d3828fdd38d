"""Test configuration.

Markers: ``gpu`` tests need an MI355X (they run through libsapphire_hip.so and are
compared with the oracle); everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and libsapphire_hip.so")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def hip():
    """The HIP library; GPU tests fail (not skip) if it is missing, and skip only when
    the machine has no GPU at all."""
    import sapphire_amd
    lib = sapphire_amd.load()
    if lib.sapphire_device_count() < 1:
        pytest.skip("no GPU on this machine")
    return lib


def close(gpu, ref, rel=1e-3, abs_=1e-4):
    """The parity tolerance for fp32 outputs: |gpu-ref| <= abs + rel*|ref|."""
    import numpy as np
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref) - (abs_ + rel * np.abs(ref))
    return float(err.max()) <= 0.0, float(np.abs(gpu - ref).max())
