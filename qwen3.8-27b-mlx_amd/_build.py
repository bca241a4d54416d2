"""Builds libgdn.so (HIP for gfx950) in-tree with hipcc."""
from __future__ import annotations

import os
import shutil
import subprocess
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libgdn.so")
SOURCES = ["gdn_api.cpp", "gdn_recurrent.hip", "gdn_commit.hip", "gdn_chunked.hip", "gdn_qlinear.hip"]

# -ffp-contract=off: the bf16 front end must round exactly as written (fma only where
#   the code asks for it with __builtin_fmaf).
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in generated code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-source additions. The chunked prefill's scan keeps its state and every MFMA result in
# VGPRs (the default heuristic puts them in AGPRs, and each elementwise step on them then
# costs a copy out and back).
SOURCE_FLAGS = {"gdn_chunked.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "gdn_qlinear.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def build(verbose: bool = False) -> str:
    """Compile every source to an object (in parallel), then link libgdn.so."""
    tmpdir = tempfile.mkdtemp(prefix="gdn_build_")
    try:
        procs, objs = [], []
        for src in SOURCES:
            obj = os.path.join(tmpdir, src + ".o")
            cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", "-o", obj, os.path.join(CSRC, src)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
            objs.append(obj)
        failed = []
        for src, pr in procs:
            out, err = pr.communicate()
            if pr.returncode != 0:
                failed.append(f"{src} ({pr.returncode}):\n{out}\n{err}")
        if failed:
            raise RuntimeError("hipcc failed: " + "\n".join(failed))
        tmp = LIB_PATH + ".tmp"
        cmd = [hipcc(), "--offload-arch=gfx950", "-fPIC", "-shared", "-o", tmp, *objs]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
        os.replace(tmp, LIB_PATH)
    finally:
        shutil.rmtree(tmpdir, ignore_errors=True)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
