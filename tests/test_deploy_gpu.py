"""GPU check of the deployment path: in a fresh process, the op runs from a
library loaded through ``ops.load_precompiled`` (sealed sidecar validated
before the library is opened, strict mode afterwards) and matches the C
oracle. The pair is exported by ``__graft_entry__.build()`` into
custom_ops_amd/deploy/.
"""
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEPLOY = os.path.join(ROOT, "custom_ops_amd", "deploy", "libmi355_fa.so")


@pytest.mark.gpu
def test_op_after_load_precompiled_matches_oracle():
    assert os.path.exists(DEPLOY) and os.path.exists(DEPLOY + ".json"), \
        "deployment pair missing: run __graft_entry__.build()"
    code = textwrap.dedent(f"""
        import os, numpy as np, torch
        from custom_ops_amd import ops, _lib
        from oracle import oracle as orc
        ops.load_precompiled("fa", {DEPLOY!r})
        assert not ops.allow_jit and ops.groups == {{"fa": "loaded"}}
        assert _lib.loaded_path() == os.path.realpath({DEPLOY!r})
        g = torch.Generator().manual_seed(7)
        B, H, Hk, Sq, Sk, d = 2, 4, 2, 77, 203, 128
        q = torch.randn(B, H, Sq, d, generator=g).bfloat16()
        k = torch.randn(B, Hk, Sk, d, generator=g).bfloat16()
        v = torch.randn(B, Hk, Sk, d, generator=g).bfloat16()
        m = torch.zeros(B, 1, Sq, Sk).masked_fill(torch.rand(B, 1, Sq, Sk, generator=g) < 0.2,
                                                  float("-inf")).bfloat16()
        m[:, :, 3, :] = float("-inf")
        out = ops.mha_fwd_with_mask(q.cuda(), k.cuda(), v.cuda(), m.cuda())
        torch.cuda.synchronize()
        out = out.float().cpu().numpy()
        ref = orc.oracle_fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                             m.float().numpy(), dtype="bf16")
        err = np.abs(out - ref)
        assert np.all(err <= 2e-2 + 2e-2 * np.abs(ref)), float(err.max())
        assert np.all(out[:, :, 3] == 0)
        print("OK", float(err.max()), flush=True)
    """)
    env = dict(os.environ, PYTHONPATH=ROOT)
    env.pop("MI355_FA_LIB", None)
    res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=240)
    assert res.returncode == 0 and "OK" in res.stdout, (res.stdout[-2000:], res.stderr[-3000:])
