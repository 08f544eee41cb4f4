"""The fused split tail (two-split launches of the compiled kernel: the last
split of each row block combines it, no combine launch) against the same
launches with the combine kernel (``Variant(fuse=-1)``), bit for bit, and
against the fp32 torch restatement of the reference op; launches of 3 and 7
splits (combine launch either way) ride along. Every case is called three
times on one workspace pool, so ticket words left by earlier launches are
exercised; the outputs of the three calls must agree bit for bit.
"""
import pytest
import torch

from tests._ref import assert_close, ref_attn_torch

CASES = [  # b, h, hk, sq, sk (Sk % 8 != 0: unaligned mask rows), d, dtype, waves
    (2, 4, 2, 300, 777, 128, torch.bfloat16, 8),
    (1, 8, 2, 513, 1000, 128, torch.float16, 4),
    (2, 16, 4, 1000, 4099, 128, torch.bfloat16, 8),
    (1, 4, 4, 256, 2048, 64, torch.bfloat16, 4),
    (3, 2, 1, 77, 333, 64, torch.float16, 8),
]


@pytest.mark.gpu
def test_fused_split_tail_matches_combine_launch(gpu):
    from custom_ops_amd import Variant, mha_fwd_with_mask
    for b, hq, hk, sq, sk, d, dt, waves in CASES:
        g = torch.Generator().manual_seed(sq * 31 + sk)
        q = (torch.randn(b, hq, sq, d, generator=g) * 0.5).to(dt).cuda()
        k = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        v = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        i = torch.arange(sq).view(sq, 1)
        j = torch.arange(sk).view(1, sk)
        m = torch.zeros(b, 1, sq, sk).masked_fill(
            (j < i) | (torch.rand(b, 1, sq, sk, generator=g) < 0.1), float("-inf"))
        m[:, :, 5, :] = float("-inf")
        m = m.to(dt).cuda()
        ref = ref_attn_torch(q, k, v, m)
        for splits in (2, 3, 7):
            res = {}
            for fuse in (0, -1):
                var = Variant(waves=waves, loop=-1, fuse=fuse)
                outs = [mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=var) for _ in range(3)]
                torch.cuda.synchronize()
                tag = (b, hq, hk, sq, sk, d, dt, waves, splits, fuse)
                for o in outs:
                    assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16)), f"repeat calls differ {tag}"
                assert_close(outs[0], ref, f"fused-tail case {tag}")
                assert bool((outs[0][:, :, 5] == 0).all())
                res[fuse] = outs[0]
            assert torch.equal(res[0].view(torch.int16), res[-1].view(torch.int16)), \
                f"fused tail differs from the combine launch {(b, hq, hk, sq, sk, d, dt, waves, splits)}"
