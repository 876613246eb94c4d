"""Runs the C++ tests of the BackendOps mirror (tests/cpp/test_backend_ops.cpp)
on the GPU as a child process and reports its per-test lines."""
import os
import subprocess

import pytest

from conftest import ROOT

BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_backend_ops")


@pytest.mark.gpu
def test_backend_ops_cpp():
    assert os.path.exists(BIN), f"{BIN} not built: run __graft_entry__.build()"
    p = subprocess.run([BIN], capture_output=True, text=True, timeout=240)
    print(p.stdout)
    print(p.stderr)
    assert p.returncode == 0, p.stdout[-4000:] + p.stderr[-2000:]
    assert "0 failed" in p.stdout
