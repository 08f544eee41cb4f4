"""The reference's examples' call pattern, unchanged, through the reference's
own import name: ``from custom_ops import ops``, then ``ops.is_available()``,
``ops.load_error()`` and ``ops.mha_fwd_with_mask(q, k, v, mask)``
(examples/basic_usage.py:24-46, gqa_example.py:22-40,
custom_mask_demo.py:28-89 of Defyli/custom_ops).

Each script runs in a fresh process with only the repository root on
``sys.path`` (as a user's checkout would be), so ``custom_ops`` must resolve to
this package by itself. Outputs are checked against the fp32 restatement of
the reference op (tests/_ref.py), at the reference tests' 2e-2 tolerance.
"""
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(code, timeout=300):
    res = subprocess.run([sys.executable, "-c", textwrap.dedent(code)], cwd=ROOT,
                         env=dict(os.environ, PYTHONPATH=ROOT), capture_output=True, text=True,
                         timeout=timeout)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-3000:])
    return res.stdout


def test_reference_import_names_resolve_here():
    """CPU: ``custom_ops`` and ``custom_ops.recsys`` are this package's objects."""
    out = _run("""
        import custom_ops, custom_ops_amd
        from custom_ops import ops, RecsysOps, FAOps, CustomOpsError
        from custom_ops.recsys import RecsysOps as R2, FAOps as F2
        assert ops is custom_ops_amd.ops and RecsysOps is custom_ops_amd.RecsysOps
        assert R2 is RecsysOps and F2 is FAOps and FAOps is custom_ops_amd.FAOps
        assert issubclass(CustomOpsError, RuntimeError)
        assert set(ops.groups) == {"fa"}
        print("ok")
    """)
    assert "ok" in out


@pytest.mark.gpu
def test_examples_call_pattern():
    out = _run("""
        import torch
        from custom_ops import ops
        from tests._ref import ref_attn_torch, assert_close

        assert torch.cuda.is_available()
        assert ops.is_available(), ops.load_error()
        assert ops.load_error() is None
        assert ops.groups == {"fa": "loaded"}

        NEG_INF = float("-inf")
        torch.manual_seed(0)

        # basic_usage.py: B2 H8 S512 d64, zero mask
        B, H, Sq, Sk, d = 2, 8, 512, 512, 64
        q = torch.randn(B, H, Sq, d, device="cuda", dtype=torch.bfloat16)
        k = torch.randn(B, H, Sk, d, device="cuda", dtype=torch.bfloat16)
        v = torch.randn(B, H, Sk, d, device="cuda", dtype=torch.bfloat16)
        mask = torch.zeros(B, 1, Sq, Sk, device="cuda", dtype=torch.bfloat16)
        out = ops.mha_fwd_with_mask(q, k, v, mask)
        assert out.shape == q.shape and out.dtype == q.dtype
        assert_close(out, ref_attn_torch(q, k, v, mask), "basic_usage")
        ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        assert (out.float() - ref.float()).abs().max().item() < 0.02

        # gqa_example.py: H16 over Hk4, unexpanded K/V
        B, H, Hk, Sq, Sk, d = 2, 16, 4, 1024, 1024, 128
        q = torch.randn(B, H, Sq, d, device="cuda", dtype=torch.bfloat16)
        k = torch.randn(B, Hk, Sk, d, device="cuda", dtype=torch.bfloat16)
        v = torch.randn(B, Hk, Sk, d, device="cuda", dtype=torch.bfloat16)
        mask = torch.zeros(B, 1, Sq, Sk, device="cuda", dtype=torch.bfloat16)
        out = ops.mha_fwd_with_mask(q, k, v, mask)
        assert_close(out, ref_attn_torch(q, k, v, mask), "gqa_example")

        # custom_mask_demo.py: causal, sliding window, padding, random 30 %
        B, H, Sq, Sk, d = 2, 8, 512, 512, 128
        q = torch.randn(B, H, Sq, d, device="cuda", dtype=torch.bfloat16)
        k = torch.randn(B, H, Sk, d, device="cuda", dtype=torch.bfloat16)
        v = torch.randn(B, H, Sk, d, device="cuda", dtype=torch.bfloat16)
        i = torch.arange(Sq, device="cuda").view(Sq, 1)
        j = torch.arange(Sk, device="cuda").view(1, Sk)
        def from_visible(visible):
            return torch.zeros(B, 1, Sq, Sk, device="cuda", dtype=torch.bfloat16).masked_fill(
                ~visible, NEG_INF)
        drop = torch.rand(B, 1, Sq, Sk, device="cuda") < 0.3
        drop[..., 0] = False
        lens = torch.tensor([Sk, Sk // 2], device="cuda")
        cases = {
            "causal": from_visible((j <= i + (Sk - Sq)).expand(B, 1, Sq, Sk)),
            "sliding_window": from_visible(((j <= i + (Sk - Sq)) & (j > i + (Sk - Sq) - 64))
                                           .expand(B, 1, Sq, Sk)),
            "padding": from_visible((j < lens.view(B, 1)).view(B, 1, 1, Sk).expand(B, 1, Sq, Sk)),
            "random_sparse": from_visible(~drop),
        }
        for name, mask in cases.items():
            out = ops.mha_fwd_with_mask(q, k, v, mask)
            assert_close(out, ref_attn_torch(q, k, v, mask), name)
            out_b = ops.mha_fwd_with_mask(q, k, v, mask, backend="auto")
            assert torch.equal(out, out_b), name
        torch.cuda.synchronize()
        print("ok")
    """)
    assert "ok" in out
