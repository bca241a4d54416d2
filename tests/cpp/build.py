"""Builds the test-side native code against libgdn.so: the C++ host-side test (test_gdn.cpp,
linked with the oracle library it checks against) and the device-math probe
(devmath_probe.hip -> libdevmath_probe.so, compiled with the library's own HIP flags).
Called by __graft_entry__.build()."""
from __future__ import annotations

import importlib.util
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
PKG_DIR = os.path.join(REPO, "qwen3.8-27b-mlx_amd")
SRC = os.path.join(HERE, "test_gdn.cpp")
BIN = os.path.join(HERE, "test_gdn")
PROBE_SRC = os.path.join(HERE, "devmath_probe.hip")
PROBE_LIB = os.path.join(HERE, "libdevmath_probe.so")


def _hipcc() -> str:
    return os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")


def _run(cmd, verbose: bool, what: str) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{what} failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")


def _library_flags():
    spec = importlib.util.spec_from_file_location("gdn_mi355x_build_flags", os.path.join(PKG_DIR, "_build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.HIPCC_FLAGS


def build(verbose: bool = False) -> str:
    _run([_hipcc(), "-std=c++17", "-O2", "-Wall", "-I", os.path.join(REPO, "include"),
          "-I", os.path.join(REPO, "oracle"), "-o", BIN, SRC,
          "-L", PKG_DIR, "-lgdn", "-L", os.path.join(REPO, "oracle"), "-loracle",
          "-Wl,-rpath,$ORIGIN/../../qwen3.8-27b-mlx_amd", "-Wl,-rpath,$ORIGIN/../../oracle"],
         verbose, "hipcc (test_gdn)")
    tmp = PROBE_LIB + ".tmp"
    _run([_hipcc(), *_library_flags(), "-shared", "-I", os.path.join(PKG_DIR, "csrc"), "-o", tmp, PROBE_SRC],
         verbose, "hipcc (devmath probe)")
    os.replace(tmp, PROBE_LIB)
    return BIN


if __name__ == "__main__":
    print(build(verbose=True))
