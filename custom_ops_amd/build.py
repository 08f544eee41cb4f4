"""Build the HIP C-ABI library ``libmi355_fa.so`` in-tree for gfx950.

hipcc cross-compiles without a GPU, so this runs on any host with ROCm.
Usage: ``python -m custom_ops_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
SRC = os.path.join(PKG_DIR, "csrc", "fa_fwd.hip")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "libmi355_fa.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)


def lib_path() -> str:
    """Library the loader opens: the in-tree build, or MI355_FA_LIB (a tuning hook
    for comparing builds of the same ABI)."""
    return os.environ.get("MI355_FA_LIB") or LIB_PATH

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (unreliable on this pool).
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def build(verbose: bool = False) -> str:
    """Compile the library (always recompiles) and return its path."""
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", SRC, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
