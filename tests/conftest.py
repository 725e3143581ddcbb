"""Shared fixtures. Tests marked `gpu` need an MI355X and the built
libndx.so; everything else runs on the CPU (the oracle, the host logic, the
C ABI's exports and its device-free paths)."""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def device():
    """The one GPU. A GPU test without a GPU fails: it must not pass on a
    fallback."""
    import naivediffusion_amd as nd
    print(f"[gpu] opening device (visible: {nd.Device.Count()})", flush=True)
    dev = nd.Device()
    print(f"[gpu] {dev.AdapterName}", flush=True)
    yield dev
    dev.Dispose()


def rel_err(actual, expected):
    """max |actual - expected| / max |expected|: the parity measure
    (QuantProbe.cs:50-57)."""
    import numpy as np
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    denom = np.max(np.abs(e))
    return float(np.max(np.abs(a - e)) / (denom if denom > 0 else 1.0))
