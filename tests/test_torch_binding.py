"""The C++ torch extension over the C ABI (custom_ops_amd/csrc/torch_binding.cpp,
built by custom_ops_amd.build as libmi355_fa_torch.so): the binding a
maintainer of the reference would add next to csrc/fa/fa_bindings.cpp, so that
the reference's Python side (recsys.py's FAOps / RecsysOps) dispatches to this
library unchanged. Each check runs in a fresh process, since the binding and
this package's Python shim register the same operator.

CPU: the library loads, registers recsys_ops::mha_fwd_with_mask with the
reference's schema (fa_bindings.cpp:37-43) and a CUDA-key kernel only.
GPU: the operator through torch.ops against the C oracle and the fp32 torch
restatement of the reference op (GQA, ragged Sk, a split plan, a fully masked
row), and an invalid GQA ratio raising the C ABI's message as a RuntimeError.
"""
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "custom_ops_amd", "libmi355_fa_torch.so")


def _run(code, timeout=300):
    res = subprocess.run([sys.executable, "-c", textwrap.dedent(code)], cwd=ROOT,
                         env=dict(os.environ, PYTHONPATH=ROOT), capture_output=True, text=True,
                         timeout=timeout)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-3000:])
    return res.stdout


@pytest.fixture(scope="module")
def binding():
    if not os.path.exists(LIB):
        from custom_ops_amd import build
        build.build_torch_binding()
    return LIB


def test_binding_registers_reference_schema(binding):
    out = _run(f"""
        import torch
        torch.ops.load_library({binding!r})
        op = torch.ops.recsys_ops.mha_fwd_with_mask
        from custom_ops_amd.fa import SCHEMA
        assert str(op.default._schema) == "recsys_ops::" + SCHEMA, op.default._schema
        has = torch._C._dispatch_has_kernel_for_dispatch_key
        assert has("recsys_ops::mha_fwd_with_mask", "CUDA")
        assert not has("recsys_ops::mha_fwd_with_mask", "CPU")
        print("ok")
    """)
    assert "ok" in out


@pytest.mark.gpu
def test_binding_parity_on_gpu(binding):
    out = _run(f"""
        import numpy as np, torch
        torch.ops.load_library({binding!r})
        from oracle import oracle as orc
        from tests._ref import ref_attn_torch, assert_close
        op = torch.ops.recsys_ops.mha_fwd_with_mask
        cases = [(1, 4, 2, 130, 301, 128, torch.bfloat16), (2, 8, 2, 64, 4099, 128, torch.bfloat16),
                 (1, 2, 1, 200, 512, 64, torch.float16)]
        for n, (b, h, hk, sq, sk, d, dt) in enumerate(cases):
            g = torch.Generator().manual_seed(7 + n)
            q = torch.randn(b, h, sq, d, generator=g).to(dt)
            k = torch.randn(b, hk, sk, d, generator=g).to(dt)
            v = torch.randn(b, hk, sk, d, generator=g).to(dt)
            m = torch.zeros(b, 1, sq, sk).masked_fill(torch.rand(b, 1, sq, sk, generator=g) < 0.1,
                                                      float("-inf"))
            m[:, :, 3, :] = float("-inf")
            m = m.to(dt)
            out = op(q.cuda(), k.cuda(), v.cuda(), m.cuda())
            torch.cuda.synchronize()
            assert_close(out, ref_attn_torch(q.cuda(), k.cuda(), v.cuda(), m.cuda()), f"case {{n}}")
            assert bool((out[:, :, 3] == 0).all())
            if n == 0:
                ref = orc.oracle_fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                     m.float().numpy(), dtype="bf16")
                err = np.abs(out.float().cpu().numpy() - ref)
                assert np.all(err <= 2e-2 + 2e-2 * np.abs(ref)), err.max()
        q = torch.randn(1, 3, 8, 64, dtype=torch.bfloat16, device="cuda")
        k = torch.randn(1, 2, 8, 64, dtype=torch.bfloat16, device="cuda")
        m = torch.zeros(1, 1, 8, 8, dtype=torch.bfloat16, device="cuda")
        try:
            op(q, k, k, m)
            raise SystemExit("an invalid GQA ratio was accepted")
        except RuntimeError as e:
            assert "divisible" in str(e), e
        print("ok")
    """)
    assert "ok" in out
