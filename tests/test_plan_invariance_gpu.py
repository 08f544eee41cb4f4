"""Plan choices that only move work between workgroups must not change a bit
of the output: GQA head packing (q-heads per workgroup), the workgroup
order (heads, heads then splits, or m-blocks fastest) and the non-temporal
K/V loads leave every row's arithmetic as it is, once
the workgroup size and the split count are fixed (packing changes the plan's
cost estimate, and a different split count or kernel legitimately rounds
differently).
"""
import pytest
import torch

CASES = [(2, 16, 4, 300, 777, torch.bfloat16, 1),
         (1, 8, 1, 513, 1000, torch.float16, 1),
         (2, 8, 2, 128, 4096, torch.bfloat16, 4)]
SETTINGS = [{}, {"pack": 1}, {"pack": 2}, {"order": 1}, {"order": 2}, {"order": 3},
            {"pack": 1, "order": 2}, {"pack": 2, "order": 3}, {"stream": 1}, {"stream": -1}]


@pytest.mark.gpu
def test_packing_and_order_are_bit_invariant(gpu):
    from custom_ops_amd import Variant, mha_fwd_with_mask
    for (b, hq, hk, sq, sk, dt, splits) in CASES:
        g = torch.Generator().manual_seed(sq * 7 + sk)
        q = torch.randn(b, hq, sq, 128, generator=g).to(dt).cuda()
        k = torch.randn(b, hk, sk, 128, generator=g).to(dt).cuda()
        v = torch.randn(b, hk, sk, 128, generator=g).to(dt).cuda()
        skm = (sk + 7) // 8 * 8
        m = torch.zeros(b, 1, sq, skm).masked_fill(torch.rand(b, 1, sq, skm, generator=g) < 0.1,
                                                   float("-inf")).to(dt).cuda()
        outs = [mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=Variant(waves=8, **s))
                for s in SETTINGS]
        torch.cuda.synchronize()
        for s, o in zip(SETTINGS, outs):
            assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16)), (s, b, hq, hk, sq, sk)
