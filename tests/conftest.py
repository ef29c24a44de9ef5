"""Shared test setup.

CPU tests (``-m "not gpu"``) exercise the oracle (oracle/liboracle.so) against
the committed golden fixtures and oracle/_ref, and check that the HIP library
loads and exports its C ABI. GPU tests (``-m gpu``) are the parity tests proper:
they call libmgprims.so through its C ABI on ``cuda:0`` and compare with the
oracle on the same seeded inputs.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "muse-glimmer-intel-serve_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and libmgprims.so")
    # the oracle is test infrastructure; build it here if this tree has none
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "oracle"], check=True,
                       stdout=subprocess.DEVNULL)


@pytest.fixture(scope="session")
def prims():
    import torch
    import mgprims
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    p = mgprims.Prims(0)
    yield p
    p.close()
