"""Plan choices that only move work between workgroups must not change a bit
of the output: GQA head packing (q-heads per workgroup) and the workgroup
order (heads or m-blocks fastest) leave every row's arithmetic as it is, once
the workgroup size and the split count are fixed (packing changes the plan's
cost estimate, and a different split count or kernel legitimately rounds
differently). Each setting runs in a fresh process; the outputs' SHA-256 must
agree.
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
    ops.ensure_loaded()
    h = hashlib.sha256()
    for (b, hq, hk, sq, sk, dt, splits) in [(2, 16, 4, 300, 777, torch.bfloat16, 1),
                                           (1, 8, 1, 513, 1000, torch.float16, 1),
                                           (2, 8, 2, 128, 4096, torch.bfloat16, 4)]:
        g = torch.Generator().manual_seed(sq * 7 + sk)
        q = torch.randn(b, hq, sq, 128, generator=g).to(dt).cuda()
        k = torch.randn(b, hk, sk, 128, generator=g).to(dt).cuda()
        v = torch.randn(b, hk, sk, 128, generator=g).to(dt).cuda()
        skm = (sk + 7) // 8 * 8
        m = torch.zeros(b, 1, sq, skm).masked_fill(torch.rand(b, 1, sq, skm, generator=g) < 0.1,
                                                   float("-inf")).to(dt).cuda()
        out = mha_fwd_with_mask(q, k, v, m, num_splits=splits)
        torch.cuda.synchronize()
        h.update(out.view(torch.int16).cpu().numpy().tobytes())
    print("HASH", h.hexdigest())
""")


def _hash(env_extra):
    env = dict(os.environ, PYTHONPATH=ROOT, MI355_FA_WAVES="8", **env_extra)
    res = subprocess.run([sys.executable, "-c", CODE], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=300)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-3000:])
    return [l for l in res.stdout.splitlines() if l.startswith("HASH")][0]


@pytest.mark.gpu
def test_packing_and_order_are_bit_invariant():
    base = _hash({})
    for extra in ({"MI355_FA_PACK": "1"}, {"MI355_FA_PACK": "2"},
                  {"MI355_FA_ORDER": "h"}, {"MI355_FA_ORDER": "m"},
                  {"MI355_FA_PACK": "1", "MI355_FA_ORDER": "m"}):
        assert _hash(extra) == base, extra
