"""Parity of every tile-loop form the library can launch for 8-wave d = 128
workgroups with 16-byte aligned mask rows, each in a fresh process (the form
is read from MI355_FA_ASM once per process):
  0  the compiled kernel
  1  the generated-assembly loop, 8 waves of 32 rows (fp16 in the default)
  2  the generated-assembly loop, 4 waves of 64 rows
  3  the generated-assembly ping-pong loop for bf16 (waves 0-3 and 4-7 one
     phase apart), fp16 as 1: the default, which the rest of the suite runs
Shapes cover one tile, ragged Sk, several tiles past the 6-tile unroll of the
ping-pong loop, GQA packing, fully masked rows and a split launch; the check is
the fp32 torch restatement of the reference op at the suite's tolerance.
"""
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CODE = textwrap.dedent("""
    import torch
    from custom_ops_amd import ops, mha_fwd_with_mask
    from tests._ref import ref_attn_torch, assert_close
    ops.ensure_loaded()
    cases = [  # b, h, hk, sq, sk, dtype, splits
        (1, 2, 2, 256, 64, torch.bfloat16, 0),
        (1, 2, 1, 256, 200, torch.bfloat16, 0),
        (2, 4, 2, 300, 777, torch.bfloat16, 0),
        (1, 8, 2, 512, 1000, torch.bfloat16, 0),
        (2, 4, 4, 256, 2048, torch.float16, 0),
        (1, 4, 4, 256, 1536, torch.bfloat16, 3),
    ]
    for b, h, hk, sq, sk, dt, splits in cases:
        g = torch.Generator().manual_seed(sk + sq)
        q = (torch.randn(b, h, sq, 128, generator=g) * 0.5).to(dt).cuda()
        k = (torch.randn(b, hk, sk, 128, generator=g) * 0.5).to(dt).cuda()
        v = (torch.randn(b, hk, sk, 128, generator=g) * 0.5).to(dt).cuda()
        skm = (sk + 7) // 8 * 8
        m = torch.zeros(b, 1, sq, skm).masked_fill(torch.rand(b, 1, sq, skm, generator=g) < 0.1,
                                                   float("-inf"))
        m[:, :, 3, :] = float("-inf")
        m = m.to(dt).cuda()[..., :skm]
        out = mha_fwd_with_mask(q, k, v, m, num_splits=splits) if splits else \\
            ops.mha_fwd_with_mask(q, k, v, m)
        torch.cuda.synchronize()
        ref = ref_attn_torch(q, k, v, m)
        assert_close(out, ref, f"form case {(b, h, hk, sq, sk, dt, splits)}")
        assert bool((out[:, :, 3] == 0).all())
    print("forms-ok")
""")


@pytest.mark.gpu
@pytest.mark.parametrize("form", ["0", "1", "2"])
def test_loop_form_parity(form):
    env = dict(os.environ, MI355_FA_ASM=form, MI355_FA_WAVES="8", PYTHONPATH=ROOT)
    res = subprocess.run([sys.executable, "-c", CODE], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0 and "forms-ok" in res.stdout, (res.stdout[-2000:], res.stderr[-3000:])
