"""Builds the C++ host-side test (test_gdn.cpp) against libgdn.so and the oracle library
it checks against. Called by __graft_entry__.build()."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
PKG_DIR = os.path.join(REPO, "qwen3.8-27b-mlx_amd")
SRC = os.path.join(HERE, "test_gdn.cpp")
BIN = os.path.join(HERE, "test_gdn")


def build(verbose: bool = False) -> str:
    hipcc = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    cmd = [hipcc, "-std=c++17", "-O2", "-Wall", "-I", os.path.join(REPO, "include"),
           "-I", os.path.join(REPO, "oracle"), "-o", BIN, SRC,
           "-L", PKG_DIR, "-lgdn", "-L", os.path.join(REPO, "oracle"), "-loracle",
           "-Wl,-rpath,$ORIGIN/../../qwen3.8-27b-mlx_amd", "-Wl,-rpath,$ORIGIN/../../oracle"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    return BIN


if __name__ == "__main__":
    print(build(verbose=True))
