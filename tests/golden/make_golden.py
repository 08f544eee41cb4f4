"""Generate tests/golden/fa_fixtures.npz.

Small seeded cases (CPU torch.Generator) covering the reference's semantic
corners: zero mask, causal, finite bias, fully masked row, trap-padded mask,
Sk = 1 and 7 (the auto-pad path), GQA 4:1, Sq = 1, d = 64 and 128, bf16 and
fp16. Inputs are stored as 16-bit patterns; the expected output is the float64
closed form softmax(q·kᵀ/√d + mask[:Sq,:Sk])·v with fully masked rows = 0
(csrc/fa/common/softmax.h:144), computed here independently of every oracle
and kernel in this repository.

Run: python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = [
    # name, dtype, B, H, Hk, Sq, Sk, d, mask kind, extra mask rows, extra mask cols
    ("zero_bf16_d64", "bf16", 1, 2, 2, 40, 48, 64, "zero", 0, 0),
    ("causal_fp16_d64", "fp16", 2, 2, 2, 33, 33, 64, "causal", 0, 0),
    ("bias_bf16_d128", "bf16", 1, 2, 2, 24, 72, 128, "bias", 0, 0),
    ("allmasked_fp16_d64", "fp16", 1, 2, 1, 17, 40, 64, "allmasked", 0, 0),
    ("trap_bf16_d64", "bf16", 1, 2, 2, 20, 40, 64, "random", 5, 8),
    ("sk1_bf16_d64", "bf16", 1, 2, 2, 9, 1, 64, "zero", 0, 0),
    ("sk7_fp16_d128", "fp16", 1, 2, 1, 12, 7, 128, "random", 0, 0),
    ("gqa4_bf16_d64", "bf16", 1, 4, 1, 16, 56, 64, "inf", 0, 0),
    ("sq1_fp16_d64", "fp16", 2, 2, 2, 1, 65, 64, "inf", 0, 0),
    ("onevisible_bf16_d64", "bf16", 1, 2, 2, 8, 24, 64, "onevisible", 0, 0),
]


def make(name, dt, B, H, Hk, Sq, Sk, d, kind, er, ec, seed):
    g = torch.Generator().manual_seed(seed)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    q = (torch.randn(B, H, Sq, d, generator=g) * 0.5).to(tdt)
    k = (torch.randn(B, Hk, Sk, d, generator=g) * 0.5).to(tdt)
    v = (torch.randn(B, Hk, Sk, d, generator=g) * 0.5).to(tdt)
    R, C = Sq + er, Sk + ec
    masked_rows = []
    if kind == "zero":
        m = torch.zeros(B, 1, R, C)
    elif kind == "causal":
        m = torch.triu(torch.full((R, C), float("-inf")), 1).expand(B, 1, R, C).clone()
    elif kind == "bias":
        m = (torch.arange(C) % 16 - 8).float().view(1, 1, 1, C).expand(B, 1, R, C).clone()
    elif kind == "random":
        m = torch.randn(B, 1, R, C, generator=g) * 0.3
    elif kind == "inf":
        m = torch.zeros(B, 1, R, C).masked_fill(torch.rand(B, 1, R, C, generator=g) < 0.2,
                                                 float("-inf"))
    elif kind == "allmasked":
        m = torch.zeros(B, 1, R, C)
        m[:, :, 0, :] = float("-inf")
        m[:, :, 9, :] = float("-inf")
        masked_rows = [0, 9]
    elif kind == "onevisible":
        m = torch.full((B, 1, R, C), float("-inf"))
        for i in range(R):
            m[:, :, i, (3 * i + 1) % Sk] = 0.0
    else:
        raise ValueError(kind)
    if ec:
        m[..., Sk:] = torch.randn(B, 1, R, ec, generator=g)   # trap: visible-looking
    m = m.to(tdt)
    qf, kf, vf, mf = (t.double().numpy() for t in (q, k, v, m))
    rep = H // Hk
    kf = np.repeat(kf, rep, axis=1)
    vf = np.repeat(vf, rep, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", qf, kf) / np.sqrt(d) + mf[:, :, :Sq, :Sk]
    mx = s.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    e = np.exp(s - mx)
    den = e.sum(-1, keepdims=True)
    p = np.where(den > 0, e / np.where(den > 0, den, 1), 0.0)
    exp = np.einsum("bhqk,bhkd->bhqd", p, vf).astype(np.float32)
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    return {
        f"{name}__q": bits(q), f"{name}__k": bits(k), f"{name}__v": bits(v),
        f"{name}__mask": bits(m), f"{name}__expected": exp,
        f"{name}__meta": np.array([1 if dt == "bf16" else 0, Sq, Sk], np.int64),
        f"{name}__masked_rows": np.array(masked_rows, np.int64),
    }


def main():
    arrays = {"names": np.array([c[0] for c in CASES])}
    for i, c in enumerate(CASES):
        arrays.update(make(*c, seed=1000 + i))
    path = os.path.join(HERE, "fa_fixtures.npz")
    np.savez_compressed(path, **arrays)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
