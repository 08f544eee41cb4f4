"""Parity of every tile-loop form the library can launch for 8-wave d = 128
workgroups with 16-byte aligned mask rows, selected per call by
``Variant(loop=...)``:
  -1 the compiled kernel
   1 the generated-assembly loop, 8 waves of 32 rows (fp16 in the default)
   2 the generated-assembly loop, 4 waves of 64 rows
   3 the generated-assembly ping-pong loop for bf16 (waves 0-3 and 4-7 one
     phase apart), fp16 as 1: the default, which the rest of the suite runs
Shapes cover one tile, ragged Sk, several tiles past the 6-tile unroll of the
ping-pong loop, GQA packing, fully masked rows and a split launch; the check is
the fp32 torch restatement of the reference op at the suite's tolerance.
"""
import pytest
import torch

from tests._ref import assert_close, ref_attn_torch

CASES = [  # b, h, hk, sq, sk, dtype, splits
    (1, 2, 2, 256, 64, torch.bfloat16, 0),
    (1, 2, 1, 256, 200, torch.bfloat16, 0),
    (2, 4, 2, 300, 777, torch.bfloat16, 0),
    (1, 8, 2, 512, 1000, torch.bfloat16, 0),
    (2, 4, 4, 256, 2048, torch.float16, 0),
    (1, 4, 4, 256, 1536, torch.bfloat16, 3),
]


@pytest.mark.gpu
@pytest.mark.parametrize("loop", [-1, 1, 2, 3])
def test_loop_form_parity(gpu, loop):
    from custom_ops_amd import Variant, mha_fwd_with_mask
    var = Variant(loop=loop, waves=8)
    for b, h, hk, sq, sk, dt, splits in CASES:
        g = torch.Generator().manual_seed(sk + sq)
        q = (torch.randn(b, h, sq, 128, generator=g) * 0.5).to(dt).cuda()
        k = (torch.randn(b, hk, sk, 128, generator=g) * 0.5).to(dt).cuda()
        v = (torch.randn(b, hk, sk, 128, generator=g) * 0.5).to(dt).cuda()
        skm = (sk + 7) // 8 * 8
        m = torch.zeros(b, 1, sq, skm).masked_fill(torch.rand(b, 1, sq, skm, generator=g) < 0.1,
                                                   float("-inf"))
        m[:, :, 3, :] = float("-inf")
        m = m.to(dt).cuda()
        out = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=var)
        torch.cuda.synchronize()
        ref = ref_attn_torch(q, k, v, m)
        assert_close(out, ref, f"loop {loop} case {(b, h, hk, sq, sk, dt, splits)}")
        assert bool((out[:, :, 3] == 0).all())
