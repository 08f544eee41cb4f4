"""bf16 masks added on the matrix core by the compiled kernel's LDS mask path
(4-wave workgroups, unaligned mask rows, d = 64), against the same launches
with the mask widened on the VALU (``Variant(mask_mfma=-1)``), and against
the fp32 torch restatement of the reference op
(tests/test_mha_fwd_with_mask.py:38-53 of the reference). The assembly loops
are off (``loop=-1``), so every 8-wave launch is the compiled kernel too.

  * masks of 0 and -inf: bit-identical to the VALU widening (the matrix core
    adds exactly 0 or -inf to each score before the QK products accumulate);
  * finite biases, -inf, bf16 finfo.min entries and a fully masked row: within
    the suite's tolerance (the selector weight is bf16(1/scale), not the fp32
    reciprocal), the fully masked row exactly 0 on both paths;
  * large finite biases (ramps over -1000..0 and +-40): the worst error of the
    matrix-core add against the fp32 restatement is pinned below the suite's
    tolerance, and is no larger than twice the VALU path's own error plus 1e-2.
"""
import pytest
import torch

from tests._ref import assert_close, ref_attn_torch

NEG = float("-inf")
CASES = [  # b, h, hk, sq, sk, d, waves, splits
    (1, 4, 4, 300, 2048, 128, 4, 1),
    (1, 8, 8, 128, 4096, 128, 4, 4),
    (2, 4, 2, 257, 777, 128, 8, 1),
    (2, 16, 4, 1000, 4099, 128, 8, 2),
    (1, 4, 4, 200, 1000, 64, 4, 1),
    (2, 4, 4, 130, 640, 64, 8, 3),
]


@pytest.mark.gpu
def test_mask_on_the_matrix_core_matches_the_valu_widening(gpu):
    from custom_ops_amd import Variant, mha_fwd_with_mask
    n = 0
    for b, hq, hk, sq, sk, d, waves, splits in CASES:
        variants = {"mfma": Variant(waves=waves, loop=-1),
                    "valu": Variant(waves=waves, loop=-1, mask_mfma=-1)}
        for kind in ("inf", "bias"):
            g = torch.Generator().manual_seed(sq * 7 + sk + d)
            q = torch.randn(b, hq, sq, d, generator=g).to(torch.bfloat16).cuda()
            k = torch.randn(b, hk, sk, d, generator=g).to(torch.bfloat16).cuda()
            v = torch.randn(b, hk, sk, d, generator=g).to(torch.bfloat16).cuda()
            m = torch.zeros(b, 1, sq, sk)
            if kind == "bias":
                m = torch.randn(b, 1, sq, sk, generator=g) * 3.0
                m[..., 3, ::5] = torch.finfo(torch.bfloat16).min
            m.masked_fill_(torch.rand(b, 1, sq, sk, generator=g) < 0.1, NEG)
            m[:, :, 7, :] = NEG
            m = m.to(torch.bfloat16).cuda()
            outs = {name: mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=var)
                    for name, var in variants.items()}
            torch.cuda.synchronize()
            ref = ref_attn_torch(q, k, v, m)
            tag = (b, hq, hk, sq, sk, d, waves, splits, kind)
            for name, o in outs.items():
                assert_close(o, ref, f"mask {name} {tag}")
                assert bool((o[:, :, 7] == 0).all()), tag
            if kind == "inf":
                assert torch.equal(outs["mfma"].view(torch.int16), outs["valu"].view(torch.int16)), tag
            n += 1
    assert n == 12


@pytest.mark.gpu
@pytest.mark.parametrize("d", [64, 128])
def test_large_finite_biases_on_the_matrix_core(gpu, d):
    """ALiBi-style biases: the matrix core scales them by bf16(1/scale), the
    reference by the fp32 reciprocal (sm89/fa_fwd_kernel.h:289); at d = 128
    that is 11.3125 against 11.3137, a relative bias of 1.1e-4 on the mask term.
    Ramps of -1000..0 per row (softmax then concentrates on the last keys) and
    +-40 noise put that bias where it matters most; the error must stay inside
    the suite's tolerance and close to the VALU widening's."""
    from custom_ops_amd import Variant, mha_fwd_with_mask
    b, h, sq, sk = 1, 4, 256, 1000
    g = torch.Generator().manual_seed(4242 + d)
    q = torch.randn(b, h, sq, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(b, h, sk, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(b, h, sk, d, generator=g).to(torch.bfloat16).cuda()
    ramp = torch.linspace(-1000.0, 0.0, sk).view(1, 1, 1, sk).expand(b, 1, sq, sk).clone()
    masks = {"ramp": ramp, "noise40": torch.randn(b, 1, sq, sk, generator=g) * 40.0,
             "ramp_fine": torch.linspace(-30.0, 0.0, sk).view(1, 1, 1, sk).expand(b, 1, sq, sk).clone()}
    for name, mf in masks.items():
        m = mf.to(torch.bfloat16).cuda()
        ref = ref_attn_torch(q, k, v, m)
        errs = {}
        for label, var in (("mfma", Variant(waves=4, loop=-1)),
                           ("valu", Variant(waves=4, loop=-1, mask_mfma=-1))):
            out = mha_fwd_with_mask(q, k, v, m, num_splits=1, variant=var)
            torch.cuda.synchronize()
            assert_close(out, ref, f"{name} {label} d{d}")
            errs[label] = (out.float() - ref).abs().max().item()
        assert errs["mfma"] <= 2 * errs["valu"] + 1e-2, (name, d, errs)
