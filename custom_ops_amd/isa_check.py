"""Checks on the gfx950 assembly of this library's own kernels, run by every
build (``custom_ops_amd.build.build``) so that a library violating them is
never produced, and by ``tests/test_isa.py``.

* M0 is written only inside the inline-assembly LDS DMA. The asm names M0 as
  a clobber; the compiler reserves M0 and does not track that clobber, so it
  must keep no value of its own in M0 anywhere in these kernels (it uses M0
  only for LDS DMA, LDS-parameter and s_sendmsg-style operations, none of
  which the kernels use outside the asm).
* No packed-FP32 arithmetic (``v_pk_{add,mul,fma}_f32``): the build disables
  the feature; this catches a flag that went missing.
* No VGPR spills and no scratch memory in any kernel (a kernel that fell
  back to scratch ran 16x slower while still passing every numeric test).
  SGPR spills are allowed only into VGPR lanes (no scratch) and only outside
  the MFMA work: every v_writelane / v_readlane of a spill VGPR lies before a
  kernel's first MFMA or after its last (a few scalar moves in the prologue
  or epilogue, never in the tile loop).
* Every kernel's register need fits its workgroup size (waves per SIMD).
* The compiled kernel (``fa_fwd_kernel``) moves nothing through AGPRs: its
  accumulators live in VGPRs, and ``v_accvgpr_read/write`` there means the
  compiler ran past its register budget and copies scores or O through AGPRs
  on every tile (VALU issue the HBM-streaming plans cannot hide). The
  assembly loops keep Q and O in AGPRs by design and are not checked.
"""
from __future__ import annotations

import re


def code_outside_asm(text: str):
    """Instruction lines of the assembly that are not inside an inline-asm block."""
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


def kernel_metadata(text: str):
    """(name, {field: value}) for every kernel in the code-object metadata."""
    meta = text[text.index("amdhsa.kernels:"):]
    for block in meta.split("\n  - ")[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        if not name:
            continue
        fields = dict(re.findall(r"\.(\w+):\s+(\d+)\s*$", block, re.M))
        yield name.group(1), fields


def kernel_body(text: str, name: str) -> list:
    """Instruction lines of one kernel (from its label to its end marker)."""
    m = re.search(rf"^{re.escape(name)}:[^\n]*\n(.*?)^\.Lfunc_end", text, re.S | re.M)
    if not m:
        return []
    return [ln.split(";", 1)[0].strip() for ln in m.group(1).splitlines()]


def sgpr_spills_in_mfma_span(text: str, name: str) -> list:
    """Spill moves (v_writelane into a spill VGPR, v_readlane out of one)
    between the kernel's first and last MFMA; empty when there are none."""
    body = kernel_body(text, name)
    if not body:
        return [f"kernel body of {name} not found"]
    mf = [i for i, c in enumerate(body) if c.startswith("v_mfma")]
    lanes = {m.group(1) for c in body for m in [re.match(r"v_writelane_b32\s+(v\d+),", c)] if m}
    if not mf or not lanes:
        return []
    lo, hi = mf[0], mf[-1]
    bad = []
    for i in range(lo, hi + 1):
        c = body[i]
        m = re.match(r"v_writelane_b32\s+(v\d+),", c) or re.match(r"v_readlane_b32\s+s\d+,\s*(v\d+),", c)
        if m and m.group(1) in lanes:
            bad.append(c)
    return bad


def violations(text: str) -> list:
    """Human-readable list of every violated property (empty when clean)."""
    out = []
    if ";;#ASMSTART" not in text:
        out.append("the LDS DMA inline assembly is missing")
    m0 = [c for c in code_outside_asm(text) if re.search(r"\bm0\b", c)]
    if m0:
        out.append(f"M0 used outside the LDS DMA asm: {m0[:5]}")
    pk = [c for c in code_outside_asm(text) if re.match(r"v_pk_(add|mul|fma)_f32\b", c)]
    if pk:
        out.append(f"packed FP32 arithmetic: {pk[:5]}")
    for name, f in kernel_metadata(text):
        if int(f.get("vgpr_spill_count", 0)) or int(f.get("private_segment_fixed_size", 0)):
            out.append(f"spills or scratch in {name}: {f}")
        elif int(f.get("sgpr_spill_count", 0)):
            bad = sgpr_spills_in_mfma_span(text, name)
            if bad:
                out.append(f"SGPR spill code inside the MFMA span of {name}: {bad[:3]}")
        if "13fa_fwd_kernelI" in name:
            agpr = [ln for ln in kernel_body(text, name) if ln.startswith("v_accvgpr_")]
            if agpr:
                out.append(f"AGPR copies in the compiled kernel {name}: {len(agpr)}, e.g. {agpr[0]}")
    if "scratch_" in "\n".join(code_outside_asm(text)):
        out.append("scratch instructions present")
    # Register need must fit the launch bounds: a SIMD holds 512 registers per
    # lane, shared by the waves of a workgroup that land on it (inline assembly
    # bound to fixed registers can push a kernel past its budget without a
    # compiler error).
    for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", text, re.S):
        nf = re.search(r"\.amdhsa_next_free_vgpr (\d+)", m.group(2))
        meta = dict(kernel_metadata(text)).get(m.group(1), {})
        wg = int(meta.get("max_flat_workgroup_size", 0) or 0)
        if nf and wg:
            per_simd = -(-wg // 256)
            if int(nf.group(1)) > 512 // per_simd:
                out.append(f"{m.group(1)} needs {nf.group(1)} registers per wave but its "
                           f"{wg}-thread workgroup puts {per_simd} waves on a SIMD")
    return out


def missed_occupancy(stderr: str) -> list:
    """hipcc's reports of kernels that missed their ``amdgpu_waves_per_eu``
    target (registers past the budget, or LDS that no longer lets the planned
    number of workgroups share a CU)."""
    return [ln.strip() for ln in stderr.splitlines() if "failed to meet occupancy target" in ln]
