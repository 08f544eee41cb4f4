"""The deep 4-wave variant (grids of at most one workgroup per CU take a third
K/V stage in dynamic LDS) against the two-stage kernel (MI355_FA_DEEP=0, read
once per process, so each setting runs in a fresh process): bit-identical
outputs over ragged key counts (the V stages past Sk are zeroed, the dynamic
one included), unaligned mask rows, d = 64, fp16, GQA packing, split and
unsplit launches, and within the suite's tolerance of the fp32 torch
restatement of the reference op.
"""
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CODE = textwrap.dedent("""
    import hashlib, os, torch
    from custom_ops_amd import ops, mha_fwd_with_mask
    from tests._ref import ref_attn_torch, assert_close
    ops.ensure_loaded()
    os.environ["MI355_FA_WAVES"] = "4"
    h = hashlib.sha256()
    cases = [  # b, h, hk, sq, sk, d, dtype, splits
        (1, 16, 16, 128, 4096, 128, torch.bfloat16, 16),
        (1, 8, 8, 100, 3001, 128, torch.bfloat16, 4),
        (2, 8, 2, 128, 2047, 128, torch.float16, 1),
        (1, 4, 4, 256, 999, 64, torch.bfloat16, 2),
        (3, 2, 1, 77, 5000, 128, torch.bfloat16, 8),
    ]
    for b, hq, hk, sq, sk, d, dt, splits in cases:
        g = torch.Generator().manual_seed(sq + sk)
        q = torch.randn(b, hq, sq, d, generator=g).to(dt).cuda()
        k = torch.randn(b, hk, sk, d, generator=g).to(dt).cuda()
        v = torch.randn(b, hk, sk, d, generator=g).to(dt).cuda()
        m = torch.randn(b, 1, sq, sk, generator=g)
        m.masked_fill_(torch.rand(b, 1, sq, sk, generator=g) < 0.1, float("-inf"))
        m[:, :, 2, :] = float("-inf")
        m = m.to(dt).cuda()
        o = mha_fwd_with_mask(q, k, v, m, num_splits=splits)
        torch.cuda.synchronize()
        assert_close(o, ref_attn_torch(q, k, v, m), f"deep case {(b, hq, hk, sq, sk, d, dt, splits)}")
        assert bool((o[:, :, 2] == 0).all())
        h.update(o.view(torch.int16).cpu().numpy().tobytes())
    print("HASH", h.hexdigest())
""")


def _hash(deep):
    env = dict(os.environ, MI355_FA_DEEP=deep, PYTHONPATH=ROOT)
    res = subprocess.run([sys.executable, "-c", CODE], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-3000:])
    return [l for l in res.stdout.splitlines() if l.startswith("HASH")][0]


@pytest.mark.gpu
def test_deep_pipeline_matches_two_stages():
    assert _hash("1") == _hash("0")
