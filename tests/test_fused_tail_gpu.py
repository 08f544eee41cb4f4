"""The fused split tail (two-split launches of the compiled kernel: the last
split of each row block combines it, no combine launch) against the same
launches with the combine kernel (MI355_FA_FUSE=0), bit for bit, and against
the fp32 torch restatement of the reference op; launches of 3 and 7 splits
(combine launch either way) ride along. Each setting runs in a fresh process
(the switch is read once per process). Every case is called three times on
one workspace, so ticket words left by earlier launches are exercised; the
outputs of the three calls must agree bit for bit.
"""
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CODE = textwrap.dedent("""
    import hashlib, torch
    from custom_ops_amd import ops, mha_fwd_with_mask
    from tests._ref import ref_attn_torch, assert_close
    ops.ensure_loaded()
    h = hashlib.sha256()
    cases = [  # b, h, hk, sq, sk (Sk % 8 != 0: unaligned mask rows), d, dtype, waves
        (2, 4, 2, 300, 777, 128, torch.bfloat16, "8"),
        (1, 8, 2, 513, 1000, 128, torch.float16, "4"),
        (2, 16, 4, 1000, 4099, 128, torch.bfloat16, "8"),
        (1, 4, 4, 256, 2048, 64, torch.bfloat16, "4"),
        (3, 2, 1, 77, 333, 64, torch.float16, "8"),
    ]
    import os
    for b, hq, hk, sq, sk, d, dt, waves in cases:
        os.environ["MI355_FA_WAVES"] = waves
        g = torch.Generator().manual_seed(sq * 31 + sk)
        q = (torch.randn(b, hq, sq, d, generator=g) * 0.5).to(dt).cuda()
        k = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        v = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        m = torch.zeros(b, 1, sq, sk)
        i = torch.arange(sq).view(sq, 1)
        j = torch.arange(sk).view(1, sk)
        m = m.masked_fill((j < i) | (torch.rand(b, 1, sq, sk, generator=g) < 0.1), float("-inf"))
        m[:, :, 5, :] = float("-inf")
        m = m.to(dt).cuda()
        ref = ref_attn_torch(q, k, v, m)
        for splits in (2, 3, 7):
            outs = [mha_fwd_with_mask(q, k, v, m, num_splits=splits) for _ in range(3)]
            torch.cuda.synchronize()
            for o in outs:
                assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16)), "repeat calls differ"
            assert_close(outs[0], ref, f"fused-tail case {(b, hq, hk, sq, sk, d, dt, waves, splits)}")
            assert bool((outs[0][:, :, 5] == 0).all())
            h.update(outs[0].view(torch.int16).cpu().numpy().tobytes())
    print("HASH", h.hexdigest())
""")


def _hash(fuse):
    env = dict(os.environ, MI355_FA_FUSE=fuse, MI355_FA_ASM="0", PYTHONPATH=ROOT)
    res = subprocess.run([sys.executable, "-c", CODE], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-3000:])
    return [l for l in res.stdout.splitlines() if l.startswith("HASH")][0]


@pytest.mark.gpu
def test_fused_split_tail_matches_combine_launch():
    assert _hash("1") == _hash("0")
