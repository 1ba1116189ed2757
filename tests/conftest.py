"""pytest configuration: the `gpu` marker and import paths.

CPU tests (`-m "not gpu"`) cover the oracle against the golden fixtures and
the eager library routines, the injection layer, and the C ABI surface of
libumic_hip.so without launching anything.  GPU tests (`-m gpu`) are the
parity tests proper: they call the HIP kernels through the C ABI and compare
with the oracle / eager torch on the same inputs.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "umic-alpamayo_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden", "umic_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X / gfx950) and libumic_hip.so")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    oracle._load()
    return oracle
