"""The row-order test of the neighbour map and the conv plan (unsorted_levels:
is row c after row a in the octree key over L levels, for every L at once)
against the keys themselves, on the CPU: tests/cpp/test_order_levels.cpp,
built by __graft_entry__.build()."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_order_levels")


def test_order_levels_match_explicit_keys():
    if not os.path.exists(BIN):
        pytest.skip("tests/cpp/test_order_levels is built by __graft_entry__.build()")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "order levels ok" in r.stdout
