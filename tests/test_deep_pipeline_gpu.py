"""The deep 4-wave variant (grids of at most one workgroup per CU take a third
K/V stage in dynamic LDS) against the two-stage kernel (``Variant(deep=-1)``):
bit-identical outputs over ragged key counts (the V stages past Sk are zeroed,
the dynamic one included), unaligned mask rows, d = 64, fp16, GQA packing,
split and unsplit launches, and within the suite's tolerance of the fp32 torch
restatement of the reference op.
"""
import pytest
import torch

from tests._ref import assert_close, ref_attn_torch

CASES = [  # b, h, hk, sq, sk, d, dtype, splits
    (1, 16, 16, 128, 4096, 128, torch.bfloat16, 16),
    (1, 8, 8, 100, 3001, 128, torch.bfloat16, 4),
    (2, 8, 2, 128, 2047, 128, torch.float16, 1),
    (1, 4, 4, 256, 999, 64, torch.bfloat16, 2),
    (3, 2, 1, 77, 5000, 128, torch.bfloat16, 8),
]


@pytest.mark.gpu
def test_deep_pipeline_matches_two_stages(gpu):
    from custom_ops_amd import Variant, mha_fwd_with_mask
    for b, hq, hk, sq, sk, d, dt, splits in CASES:
        g = torch.Generator().manual_seed(sq + sk)
        q = torch.randn(b, hq, sq, d, generator=g).to(dt).cuda()
        k = torch.randn(b, hk, sk, d, generator=g).to(dt).cuda()
        v = torch.randn(b, hk, sk, d, generator=g).to(dt).cuda()
        m = torch.randn(b, 1, sq, sk, generator=g)
        m.masked_fill_(torch.rand(b, 1, sq, sk, generator=g) < 0.1, float("-inf"))
        m[:, :, 2, :] = float("-inf")
        m = m.to(dt).cuda()
        tag = (b, hq, hk, sq, sk, d, dt, splits)
        deep = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=Variant(waves=4))
        two = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=Variant(waves=4, deep=-1))
        torch.cuda.synchronize()
        assert_close(deep, ref_attn_torch(q, k, v, m), f"deep case {tag}")
        assert bool((deep[:, :, 2] == 0).all())
        assert torch.equal(deep.view(torch.int16), two.view(torch.int16)), f"deep != two stages {tag}"
