"""Runs the C++ host-side test (tests/cpp/test_gdn.cpp, built by __graft_entry__.build())
on the GPU: gdn.hpp's run / DeltaCache against the oracle, in the reference's self-test
style (cpp/src/tests.cpp:196-243)."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_gdn")


def test_cpp_host_layer():
    print("[case] C++ host test tests/cpp/test_gdn", flush=True)
    assert os.path.exists(BIN), "tests/cpp/test_gdn is not built: run __graft_entry__.build()"
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=180)
    print(res.stdout[-4000:], flush=True)
    assert "[skip]" not in res.stdout, "the C++ test found no gfx950 device"
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    assert "[FAIL]" not in res.stdout
