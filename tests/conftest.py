"""Test configuration: the `gpu` marker, repo-root imports, shared fixtures.

`-m "not gpu"` runs the oracle-vs-golden checks, the host logic and the C-ABI
export checks on the CPU; `-m gpu` runs the parity tests through the C ABI on
an MI355X.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    with np.load(os.path.join(ROOT, "tests", "golden", "golden.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def vh():
    """The C ABI, initialised on device 0 (GPU tests only)."""
    from vearo_amd import _abi

    _abi.init(0)
    return _abi


def pytest_sessionfinish(session, exitstatus):
    """Writes the parity statistics of every assert_parity call (tests/parity.py)
    to the file VH_PARITY_REPORT names, if set."""
    path = os.environ.get("VH_PARITY_REPORT")
    if not path:
        return
    import json

    import parity

    with open(path, "w") as f:
        json.dump(parity.REPORT, f, indent=1)
