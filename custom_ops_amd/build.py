"""Build the HIP C-ABI library ``libmi355_fa.so`` in-tree for gfx950.

hipcc cross-compiles without a GPU, so this runs on any host with ROCm.
Usage: ``python -m custom_ops_amd.build`` (or ``__graft_entry__.build()``).
Every build also checks the gfx950 assembly it produced
(``custom_ops_amd.isa_check``) and refuses to install a library that
violates those properties.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
import tempfile

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


def compile_checked(out_path: str, flags=None, verbose: bool = False) -> str:
    """Compile SRC into ``out_path`` (atomically) after checking the device
    assembly of that same compilation; raise RuntimeError on either failure."""
    from .isa_check import missed_occupancy, violations
    flags = list(HIPCC_FLAGS if flags is None else flags)
    with tempfile.TemporaryDirectory(prefix="mi355fa-build-") as tmp:
        product = os.path.join(tmp, os.path.basename(out_path))
        cmd = [hipcc(), *flags, f"-I{INCLUDE}", SRC, "-o", product, "-save-temps=obj"]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True, cwd=tmp)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
        # A kernel that misses its amdgpu_waves_per_eu target has lost the
        # occupancy its tiling was designed for (registers past the budget,
        # or LDS that no longer lets two workgroups share a CU).
        missed = missed_occupancy(res.stderr)
        if missed:
            raise RuntimeError("occupancy target missed; library not installed:\n" + "\n".join(missed[:8]))
        asm = sorted(glob.glob(os.path.join(tmp, "*amdgcn-amd-amdhsa*.s")))
        if not asm:
            raise RuntimeError("hipcc left no device assembly to check")
        bad = []
        for path in asm:
            with open(path) as f:
                bad += [f"{os.path.basename(path)}: {v}" for v in violations(f.read())]
        if bad:
            raise RuntimeError("device assembly check failed; library not installed:\n"
                               + "\n".join(bad))
        tmp_out = out_path + ".tmp"
        shutil.copyfile(product, tmp_out)
        os.chmod(tmp_out, 0o755)
        os.replace(tmp_out, out_path)
    return out_path


TORCH_BINDING_SRC = os.path.join(PKG_DIR, "csrc", "torch_binding.cpp")
TORCH_BINDING_PATH = os.path.join(PKG_DIR, "libmi355_fa_torch.so")


def build_torch_binding(verbose: bool = False) -> str:
    """Compile the C++ torch extension over the C ABI (csrc/torch_binding.cpp:
    the reference-style TORCH_LIBRARY binding) against this PyTorch-ROCm, linked
    to libmi355_fa.so next to it. Host code only, so the host compiler builds it."""
    import torch
    tdir = os.path.dirname(torch.__file__)
    abi = int(torch.compiled_with_cxx11_abi())
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-DUSE_ROCM", "-D__HIP_PLATFORM_AMD__",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-I{tdir}/include",
           f"-I{tdir}/include/torch/csrc/api/include", "-I/opt/rocm/include", f"-I{INCLUDE}",
           TORCH_BINDING_SRC, "-o", TORCH_BINDING_PATH + ".tmp",
           f"-L{tdir}/lib", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-L/opt/rocm/lib", "-lamdhip64", f"-L{PKG_DIR}", "-lmi355_fa", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch binding build failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(TORCH_BINDING_PATH + ".tmp", TORCH_BINDING_PATH)
    return TORCH_BINDING_PATH


def build(verbose: bool = False) -> str:
    """Compile the library (always recompiles) and the C++ torch binding over
    it; return the library's path."""
    out = compile_checked(LIB_PATH, verbose=verbose)
    build_torch_binding(verbose=verbose)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
