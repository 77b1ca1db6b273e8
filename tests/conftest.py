"""Shared pytest setup: import paths and the `gpu` marker.

Tests marked `gpu` need an MI355X and the built libqmla.so; everything else
runs on the CPU (oracle checks, header/ABI checks)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "qmoe-rs_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libqmla.so")


@pytest.fixture(scope="session")
def golden():
    return np.load(os.path.join(ROOT, "tests", "golden", "golden.npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def qmla_gpu():
    """The qmla binding with a live GPU; fails (never falls back) otherwise."""
    import qmla
    dev, cus, arch = qmla.device_info()
    assert cus > 0, "no GPU visible"
    print(f"[gpu] device {dev}: {arch}, {cus} CUs", flush=True)
    return qmla
