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
row); and every argument check, which must raise the reference's RuntimeError
text (csrc/fa/fa_fwd_op.cu:53-108) before anything is launched, for the same
inputs for which this package's Python shim raises it.
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


# (description, builder of (q, k, v, mask) on the GPU, expected message). Each
# input breaks exactly one rule; the binding must stop at that rule's check.
BAD_INPUTS = """
def bad_inputs():
    import torch
    bf, dev = torch.bfloat16, "cuda"
    def t(*shape, dtype=bf, device=dev):
        return torch.zeros(*shape, dtype=dtype, device=device)
    q, k, m = t(1, 4, 8, 64), t(1, 2, 8, 64), t(1, 1, 8, 8)
    return [
        ("q on the host", (t(1, 4, 8, 64, device="cpu"), k, k, m), "q must be a CUDA tensor"),
        ("mask on the host", (q, k, k, t(1, 1, 8, 8, device="cpu")), "mask must be a CUDA tensor"),
        ("fp32", (t(1, 4, 8, 64, dtype=torch.float32), t(1, 2, 8, 64, dtype=torch.float32),
                  t(1, 2, 8, 64, dtype=torch.float32), t(1, 1, 8, 8, dtype=torch.float32)),
         "q must be float16 or bfloat16"),
        ("fp16 k", (q, t(1, 2, 8, 64, dtype=torch.float16), k, m), "k dtype must match q"),
        ("fp16 v", (q, k, t(1, 2, 8, 64, dtype=torch.float16), m), "v dtype must match q"),
        ("fp16 mask", (q, k, k, t(1, 1, 8, 8, dtype=torch.float16)), "mask dtype must match q"),
        ("q transposed", (t(1, 4, 64, 8).transpose(2, 3), k, k, m), "q must be contiguous"),
        ("k sliced", (q, t(1, 2, 8, 128)[..., :64], k, m), "k must be contiguous"),
        ("v strided heads", (q, k, t(1, 4, 8, 64)[:, ::2], m), "v must be contiguous"),
        ("mask transposed", (q, k, k, t(1, 1, 8, 8).transpose(2, 3)), "mask must be contiguous"),
        ("q 3-D", (t(4, 8, 64), k, k, m), "q must be 4D"),
        ("mask 3-D", (q, k, k, t(1, 8, 8)), "mask must be 4D"),
        ("k batch", (q, t(2, 2, 8, 64), k, m), "Batch size mismatch"),
        ("v batch", (q, k, t(2, 2, 8, 64), m), "Batch size mismatch"),
        ("mask batch", (q, k, k, t(2, 1, 8, 8)), "Batch size mismatch"),
        ("k head_dim", (q, t(1, 2, 8, 128), k, m), "head_dim mismatch between q/k/v"),
        ("v head_dim", (q, k, t(1, 2, 8, 128), m), "head_dim mismatch between q/k/v"),
        ("v seqlen", (q, k, t(1, 2, 9, 64), m), "seqlen_k mismatch between k/v"),
        ("GQA ratio", (t(1, 3, 8, 64), k, k, m), "n_heads must be divisible by n_kv_heads"),
        ("head_dim 96", (t(1, 4, 8, 96), t(1, 2, 8, 96), t(1, 2, 8, 96), m),
         "Only head_dim=64 or head_dim=128 is supported"),
        ("mask heads", (q, k, k, t(1, 2, 8, 8)), "mask shape must be"),
        ("mask rows", (q, k, k, t(1, 1, 7, 8)), "mask shape must be"),
        ("mask cols", (q, k, k, t(1, 1, 8, 7)), "mask shape must be"),
        ("v heads", (q, k, t(1, 4, 8, 64), m), "n_kv_heads mismatch between k/v"),
    ]
"""


@pytest.mark.gpu
def test_binding_rejects_like_reference(binding):
    """Every argument check of the binding raises the reference's message, and
    the Python shim (custom_ops_amd.fa.validate) raises the same one for the
    same inputs; nothing is launched for any of them."""
    out = _run(BAD_INPUTS + f"""
import re, torch
torch.ops.load_library({binding!r})
from custom_ops_amd import fa
op = torch.ops.recsys_ops.mha_fwd_with_mask
for name, args, msg in bad_inputs():
    for label, fn in (("binding", lambda: op(*args)), ("shim", lambda: fa.validate(*args))):
        try:
            fn()
        except RuntimeError as e:
            assert msg in str(e), (label, name, str(e)[:300])
        else:
            raise SystemExit(f"{{label}} accepted {{name}}")
torch.cuda.synchronize()
print("ok", len(bad_inputs()))
""")
    assert "ok 24" in out
