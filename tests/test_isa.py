"""CPU checks on the gfx950 assembly of this build's own kernels (hipcc
cross-compiles without a GPU), through the same checker every build runs
(custom_ops_amd/isa_check.py): M0 only inside the LDS-DMA inline assembly, no
packed FP32, no spills or scratch. Also pins that the checker itself catches
each kind of violation, so a build that breaks them cannot be installed.
"""
import subprocess

import pytest

from custom_ops_amd import build
from custom_ops_amd.isa_check import code_outside_asm, kernel_metadata, violations


@pytest.fixture(scope="module")
def isa(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "fa_fwd.s"
    flags = [f for f in build.HIPCC_FLAGS if f not in ("-fPIC", "-shared")]
    cmd = [build.hipcc(), *flags, "--cuda-device-only", "-S", f"-I{build.INCLUDE}", build.SRC,
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-3000:]
    return out.read_text()


def test_build_assembly_is_clean(isa):
    assert violations(isa) == []


def test_every_variant_present(isa):
    kernels = [k for k, _ in kernel_metadata(isa)]
    assert len(kernels) >= 40, kernels


def test_m0_only_inside_the_lds_dma_asm(isa):
    assert ";;#ASMSTART" in isa
    assert not [c for c in code_outside_asm(isa) if "m0" in c.split()]


_FAKE = """\
\t;;#ASMSTART
\ts_mov_b32 m0, s1
\tbuffer_load_dwordx4 v1, s[4:7], 0 offen lds
\t;;#ASMEND
{body}
amdhsa.kernels:
  - .name:           k
    .private_segment_fixed_size: {scratch}
    .sgpr_spill_count: 0
    .vgpr_spill_count: {spill}
"""


@pytest.mark.parametrize("body,scratch,spill,expect", [
    ("\tv_add_f32 v1, v2, v3", 0, 0, None),
    ("\ts_mov_b32 m0, s2", 0, 0, "M0 used outside"),
    ("\tv_pk_fma_f32 v[0:1], v[2:3], v[4:5], v[6:7]", 0, 0, "packed FP32"),
    ("\tv_add_f32 v1, v2, v3", 16, 0, "spills or scratch"),
    ("\tv_add_f32 v1, v2, v3", 0, 3, "spills or scratch"),
])
def test_checker_catches_each_violation(body, scratch, spill, expect):
    found = violations(_FAKE.format(body=body, scratch=scratch, spill=spill))
    if expect is None:
        assert found == []
    else:
        assert any(expect in v for v in found), found
