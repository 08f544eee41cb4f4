"""CPU checks on the gfx950 assembly of this build's own kernels (hipcc
cross-compiles without a GPU). They pin properties the GPU tests cannot see
directly and that a compiler or source change can silently break:

* M0 is written only inside the inline-assembly LDS DMA (which names it as a
  clobber): the compiler must not keep a value of its own in M0 across it;
* no packed-FP32 arithmetic (the build disables it);
* no register spills and no scratch memory in any kernel (a kernel that fell
  back to scratch ran 16x slower while still passing every numeric test).
"""
import os
import re
import subprocess

import pytest

from custom_ops_amd import build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def isa(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "fa_fwd.s"
    flags = [f for f in build.HIPCC_FLAGS if f not in ("-fPIC", "-shared")]
    cmd = [build.hipcc(), *flags, "--cuda-device-only", "-S", f"-I{build.INCLUDE}", build.SRC,
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-3000:]
    return out.read_text()


def _code_outside_asm(text):
    inside = False
    for line in text.splitlines():
        if ";;#ASMSTART" in line:
            inside = True
            continue
        if ";;#ASMEND" in line:
            inside = False
            continue
        code = line.split(";", 1)[0].strip()
        if not inside and code:
            yield code


def _kernel_metadata(text):
    """(name, {field: value}) for every kernel in the code-object metadata."""
    meta = text[text.index("amdhsa.kernels:"):]
    for block in meta.split("\n  - ")[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        if not name:
            continue
        fields = dict(re.findall(r"\.(\w+):\s+(\d+)\s*$", block, re.M))
        yield name.group(1), fields


def test_m0_only_inside_the_lds_dma_asm(isa):
    assert ";;#ASMSTART" in isa, "the LDS DMA inline assembly is missing"
    offenders = [c for c in _code_outside_asm(isa) if re.search(r"\bm0\b", c)]
    assert not offenders, offenders[:10]


def test_no_packed_fp32_arithmetic(isa):
    offenders = [c for c in _code_outside_asm(isa)
                 if re.match(r"v_pk_(add|mul|fma)_f32\b", c)]
    assert not offenders, offenders[:10]


def test_no_spills_or_scratch(isa):
    kernels = list(_kernel_metadata(isa))
    assert len(kernels) >= 40, [k for k, _ in kernels]
    bad = {name: f for name, f in kernels
           if int(f.get("vgpr_spill_count", 0)) or int(f.get("sgpr_spill_count", 0))
           or int(f.get("private_segment_fixed_size", 0))}
    assert not bad, bad
    assert "scratch_" not in isa
