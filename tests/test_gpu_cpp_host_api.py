"""Runs the C++ host-mirror test program (tests/cpp/test_host_api.cpp, built by
__graft_entry__.build()) on the GPU."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_host_api")


def test_cpp_host_api():
    assert os.path.exists(BIN), "build the C++ host test with __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "host api ok" in r.stdout
