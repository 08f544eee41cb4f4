"""bf16 masks added on the matrix core by the compiled kernel's LDS mask path
(4-wave workgroups, unaligned mask rows, d = 64; MI355_FA_MASK_MFMA, read at
every launch, switches it off): against the same launches with the mask
widened on the VALU, and against the fp32 torch restatement of the reference
op (tests/test_mha_fwd_with_mask.py:38-53 of the reference).

  * masks of 0 and -inf: bit-identical to the VALU widening (the matrix core
    adds exactly 0 or -inf to each score before the QK products accumulate);
  * finite biases, -inf, bf16 finfo.min entries and a fully masked row: within
    the suite's tolerance (the selector weight is bf16(1/scale), not the fp32
    reciprocal), the fully masked row exactly 0 on both paths.

Runs in a fresh process with the assembly loops off (MI355_FA_ASM=0, read
once per process), so every 8-wave launch is the compiled kernel too.
"""
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CODE = textwrap.dedent("""
    import os, torch
    from custom_ops_amd import ops, mha_fwd_with_mask
    from tests._ref import ref_attn_torch, assert_close
    ops.ensure_loaded()
    NEG = float("-inf")
    cases = [  # b, h, hk, sq, sk, d, waves, splits
        (1, 4, 4, 300, 2048, 128, "4", 1),
        (1, 8, 8, 128, 4096, 128, "4", 4),
        (2, 4, 2, 257, 777, 128, "8", 1),
        (2, 16, 4, 1000, 4099, 128, "8", 2),
        (1, 4, 4, 200, 1000, 64, "4", 1),
        (2, 4, 4, 130, 640, 64, "8", 3),
    ]
    n = 0
    for b, hq, hk, sq, sk, d, waves, splits in cases:
        os.environ["MI355_FA_WAVES"] = waves
        for kind in ("inf", "bias"):
            g = torch.Generator().manual_seed(sq * 7 + sk + d)
            q = torch.randn(b, hq, sq, d, generator=g).to(torch.bfloat16).cuda()
            k = torch.randn(b, hk, sk, d, generator=g).to(torch.bfloat16).cuda()
            v = torch.randn(b, hk, sk, d, generator=g).to(torch.bfloat16).cuda()
            m = torch.zeros(b, 1, sq, sk)
            if kind == "bias":
                m = torch.randn(b, 1, sq, sk, generator=g) * 3.0
                m[..., 3, ::5] = torch.finfo(torch.bfloat16).min
            m.masked_fill_(torch.rand(b, 1, sq, sk, generator=g) < 0.1, NEG)
            m[:, :, 7, :] = NEG
            m = m.to(torch.bfloat16).cuda()
            outs = {}
            for mm in ("1", "0"):
                os.environ["MI355_FA_MASK_MFMA"] = mm
                outs[mm] = mha_fwd_with_mask(q, k, v, m, num_splits=splits)
            torch.cuda.synchronize()
            ref = ref_attn_torch(q, k, v, m)
            tag = (b, hq, hk, sq, sk, d, waves, splits, kind)
            for mm, o in outs.items():
                assert_close(o, ref, f"mask-mfma {mm} {tag}")
                assert bool((o[:, :, 7] == 0).all()), tag
            if kind == "inf":
                assert torch.equal(outs["1"].view(torch.int16), outs["0"].view(torch.int16)), tag
            n += 1
    print("CASES", n)
""")


@pytest.mark.gpu
def test_mask_on_the_matrix_core_matches_the_valu_widening():
    env = dict(os.environ, MI355_FA_ASM="0", PYTHONPATH=ROOT)
    res = subprocess.run([sys.executable, "-c", CODE], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-3000:])
    assert "CASES 12" in res.stdout
