"""CPU checks on the gfx950 assembly of this build's own kernels (hipcc
cross-compiles without a GPU), through the same checker every build runs
(custom_ops_amd/isa_check.py): M0 only inside the LDS-DMA inline assembly, no
packed FP32, no VGPR spills or scratch, SGPR spills only into VGPR lanes
outside the MFMA span. Also pins that the checker itself catches
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


_SPILL = """\
\t;;#ASMSTART
\ts_mov_b32 m0, s1
\t;;#ASMEND
k:                                      ; @k
{pre}
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
{mid}
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
{post}
\ts_endpgm
.Lfunc_end0:
amdhsa.kernels:
  - .name:           k
    .private_segment_fixed_size: 0
    .sgpr_spill_count: 1
    .vgpr_spill_count: 0
"""

_WL = "\tv_writelane_b32 v231, s80, 0"
_RL = "\tv_readlane_b32 s80, v231, 0"


@pytest.mark.parametrize("pre,mid,post,ok", [
    (_WL, "", _RL, True),                      # spilled before the MFMA span, restored after
    (_WL + "\n" + _RL, "", "", True),         # both in the prologue
    (_WL, _RL, "", False),                     # restored inside the span
    ("", _WL, _RL, False),                     # spilled inside the span
    (_WL, "\tv_readlane_b32 s2, v18, 16", _RL, True),   # a readlane of another VGPR (a reduction)
])
def test_checker_sgpr_spills_only_outside_the_mfma_span(pre, mid, post, ok):
    found = [v for v in violations(_SPILL.format(pre=pre, mid=mid, post=post)) if "SGPR spill" in v]
    assert (found == []) == ok, found


_AGPR = """\
	;;#ASMSTART
	s_mov_b32 m0, s1
	;;#ASMEND
{name}:                                      ; @k
	v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
{body}
	s_endpgm
.Lfunc_end0:
amdhsa.kernels:
  - .name:           {name}
    .private_segment_fixed_size: 0
    .sgpr_spill_count: 0
    .vgpr_spill_count: 0
"""


@pytest.mark.parametrize("name,body,ok", [
    ("_ZN7mi355fa13fa_fwd_kernelILi128ELb1ELb1ELb1ELi4EEEvNS_7KParamsE", "\tv_mul_f32 v1, v2, v3", True),
    ("_ZN7mi355fa13fa_fwd_kernelILi128ELb1ELb1ELb1ELi4EEEvNS_7KParamsE", "\tv_accvgpr_read_b32 v1, a7", False),
    ("_ZN7mi355fa17fa_fwd_kernel_asmILi1ELb1ELb0EEEvNS_7KParamsE", "\tv_accvgpr_read_b32 v1, a7", True),
])
def test_checker_catches_agpr_copies_in_the_compiled_kernel(name, body, ok):
    found = [v for v in violations(_AGPR.format(name=name, body=body)) if "AGPR copies" in v]
    assert (found == []) == ok, found


_REGFIT = """\
\t.amdhsa_kernel k
\t\t.amdhsa_next_free_vgpr {nf}
\t.end_amdhsa_kernel
amdhsa.kernels:
  - .name:           k
    .max_flat_workgroup_size: {wg}
    .private_segment_fixed_size: 0
    .sgpr_spill_count: 0
    .vgpr_spill_count: 0
"""


@pytest.mark.parametrize("nf,wg,ok", [(256, 512, True), (337, 512, False), (420, 256, True),
                                      (513, 64, False)])
def test_checker_catches_register_overcommit(nf, wg, ok):
    found = [v for v in violations(_REGFIT.format(nf=nf, wg=wg)) if "registers per wave" in v]
    assert (found == []) == ok, found


def test_generated_loop_is_current():
    """fa_loop.inc is generated by gen_fa_loop.py; a hand edit or a stale copy
    of either one fails here."""
    import os
    import sys
    gen = os.path.join(os.path.dirname(build.SRC), "gen_fa_loop.py")
    res = subprocess.run([sys.executable, gen, "--check"], timeout=300)
    assert res.returncode == 0, "fa_loop.inc differs from gen_fa_loop.py's output"


def _declared_and_written(inc):
    """Per generated loop in fa_loop.inc: the registers its asm statement
    declares (outputs, in/out operands, clobbers) and the ones its text writes
    (first operand of VALU / LDS / global loads into VGPRs, SALU results)."""
    import re
    out = {}
    for m in re.finditer(r"#define MI355_(\w+)_LOOP_(BF16|F16) ", inc):
        pre, dt = m.group(1), m.group(2)
        end = inc.find("\n#define", m.end())
        body = inc[m.end():end if end > 0 else len(inc)]

        def mac(kind):
            k = inc.index(f"#define MI355_{pre}_{kind}_{dt} ")
            return inc[k:inc.find("\n", k)]
        decl = {"v": set(), "s": set()}
        for kind in ("OUTPUTS", "CLOBBERS"):
            t = mac(kind)
            for f, a, b in re.findall(r"([vs])\[(\d+):(\d+)\]", t):
                decl[f] |= set(range(int(a), int(b) + 1))
            for f, a in re.findall(r'"([vs])(\d+)"', t) + re.findall(r"\{([vs])(\d+)\}", t):
                decl[f].add(int(a))
        wrote = {"v": set(), "s": set()}
        for ins in re.findall(r'"([^"]*)\\n\\t"', body):
            toks = ins.strip().split(None, 1)
            if len(toks) < 2 or toks[0].endswith(":"):
                continue
            op, rest = toks
            if op.startswith(("v_cmp", "s_cmp", "s_cbranch", "s_waitcnt", "s_nop", "s_barrier", "s_branch",
                              "v_accvgpr_write", "global_store", "buffer_store", "ds_write", "s_setprio")):
                continue
            if op.startswith("buffer_load") and rest.rstrip().endswith(" lds"):
                continue            # LDS DMA: writes no register
            dst = rest.split(",")[0].strip()
            r = re.match(r"([vs])\[(\d+):(\d+)\]$", dst)
            if r:
                wrote[r.group(1)] |= set(range(int(r.group(2)), int(r.group(3)) + 1))
                continue
            r = re.match(r"([vs])(\d+)$", dst)
            if r:
                wrote[r.group(1)].add(int(r.group(2)))
        out[f"{pre}_{dt}"] = (decl, wrote)
    return out


def test_loops_declare_every_register_they_write():
    """A register the loop text writes but its asm statement does not declare
    can hold a compiler value (an address, a loop bound) across the statement."""
    import os
    inc = open(os.path.join(os.path.dirname(build.SRC), "fa_loop.inc")).read()
    loops = _declared_and_written(inc)
    assert {"W32_BF16", "W32_F16", "W64_BF16", "W64_F16", "PP_BF16"} <= set(loops)
    for name, (decl, wrote) in loops.items():
        for f in ("v", "s"):
            assert not (wrote[f] - decl[f]), (name, f, sorted(wrote[f] - decl[f])[:16])


def test_register_declaration_check_catches_an_undeclared_write():
    inc = ('#define MI355_X_LOOP_BF16 "v_mov_b32 v7, 0\\n\\t" "s_mov_b32 s70, 0\\n\\t"\n'
           '#define MI355_X_OUTPUTS_BF16 "={v[0:3]}"(o)\n'
           '#define MI355_X_CLOBBERS_BF16 "v6", "s69"\n')
    decl, wrote = _declared_and_written(inc)["X_BF16"]
    assert wrote["v"] - decl["v"] == {7} and wrote["s"] - decl["s"] == {70}


def test_missed_occupancy_target_is_reported():
    from custom_ops_amd.isa_check import missed_occupancy
    err = ("warning: <unknown>:0:0: failed to meet occupancy target given by 'amdgpu-waves-per-eu' in "
           "'k': desired occupancy was 2, final occupancy is 1 [-Wpass-failed]\n"
           "warning: inline asm clobber list contains reserved registers: M0\n")
    assert len(missed_occupancy(err)) == 1
    assert missed_occupancy("warning: inline asm clobber list contains reserved registers: M0\n") == []



def _functions(isa):
    """(name, lines) of every kernel body in the assembly."""
    import re
    out, name, body = [], None, []
    for line in isa.splitlines():
        m = re.match(r"^(_Z\w+):", line)
        if m:
            name, body = m.group(1), []
            continue
        if name is None:
            continue
        body.append(line.strip())
        if line.strip().startswith("s_endpgm"):
            out.append((name, body))
            name = None
    return out


def _fused_tail_ordering(body):
    """Problems with the fused split tail's ordering in one kernel body (empty
    when it is right, or when the kernel has no ticket atomic)."""
    code = [l for l in body if l and not l.startswith(";") and not l.startswith(".")]
    cas = [i for i, l in enumerate(code) if "atomic_cmpswap" in l]
    bad = []
    for i in cas:
        bar = max((j for j in range(i) if code[j].startswith("s_barrier")), default=None)
        if bar is None:
            bad.append("no s_barrier before the ticket CAS")
            continue
        wait = max((j for j in range(bar) if code[j].startswith("s_waitcnt") and "vmcnt(0)" in code[j]),
                   default=None)
        if wait is None:
            bad.append("no s_waitcnt vmcnt(0) before the barrier that precedes the CAS")
            continue
        if any(code[j].startswith(("buffer_store", "global_store", "flat_store")) for j in range(wait, i)):
            bad.append("a store between the vmcnt(0) wait and the CAS")
        last = max((j for j in range(wait) if code[j].startswith("buffer_store")), default=None)
        if last is None or "sc1" not in code[last]:
            bad.append("the last partial store before the wait is not sc1")
        for l in code[i + 1:]:
            if l.startswith("buffer_load") and "sc1" not in l:
                bad.append(f"buffer load after the CAS without sc1: {l}")
    return bad


def test_fused_tail_ordering_in_the_assembly(isa):
    """The fused split tail's release and acquire are built from instruction
    order and cache-policy bits (see ticket_arrive in csrc/fa_fwd.hip): every
    kernel with a ticket CAS must show, in its assembly, an s_waitcnt vmcnt(0)
    and an s_barrier between its last (sc1) partial store and the CAS, no store
    in between, and sc1 on every buffer load after the CAS."""
    checked = 0
    for name, body in _functions(isa):
        if not any("atomic_cmpswap" in l for l in body):
            continue
        checked += 1
        assert not _fused_tail_ordering(body), (name, _fused_tail_ordering(body))
    assert checked >= 4, checked


@pytest.mark.parametrize("body,ok", [
    (["buffer_store_dwordx4 v[1:4], v0, s[4:7], 0 offen sc1", "s_waitcnt vmcnt(0)", "s_barrier",
      "flat_atomic_cmpswap_x2 v[2:3], v[4:5], v[6:9] sc0", "buffer_load_dwordx4 v[1:4], v0, s[4:7], 0 offen sc1",
      "s_endpgm"], True),
    (["buffer_store_dwordx4 v[1:4], v0, s[4:7], 0 offen sc1", "s_barrier",
      "flat_atomic_cmpswap_x2 v[2:3], v[4:5], v[6:9] sc0", "s_endpgm"], False),
    (["buffer_store_dwordx4 v[1:4], v0, s[4:7], 0 offen", "s_waitcnt vmcnt(0)", "s_barrier",
      "flat_atomic_cmpswap_x2 v[2:3], v[4:5], v[6:9] sc0", "s_endpgm"], False),
    (["buffer_store_dwordx4 v[1:4], v0, s[4:7], 0 offen sc1", "s_waitcnt vmcnt(0)", "s_barrier",
      "flat_atomic_cmpswap_x2 v[2:3], v[4:5], v[6:9] sc0", "buffer_load_dwordx4 v[1:4], v0, s[4:7], 0 offen",
      "s_endpgm"], False),
])
def test_fused_tail_ordering_check_catches_violations(body, ok):
    assert (not _fused_tail_ordering(body)) == ok
