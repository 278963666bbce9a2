import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ref_vectors():
    with open(GOLDEN / "reference_vectors.json") as f:
        return json.load(f)


@pytest.fixture(scope="session")
def oracle():
    import oracle as o  # oracle/oracle.py (test infrastructure)
    return o


@pytest.fixture(scope="session")
def native():
    """libsilgpu through ctypes, initialised on device 0.  Raises (no skip)
    when the library or the GPU is missing: GPU tests must not pass silently."""
    from silarray_amd import _native as nat
    nat.init()
    info = nat.device_info()
    assert info["arch"].startswith("gfx950"), info
    return nat


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)
