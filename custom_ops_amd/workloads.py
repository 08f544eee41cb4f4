"""Synthetic workloads for the five benchmark configurations of ``mha_fwd_with_mask``.

All inputs come from ONE CPU ``torch.Generator`` seeded 42, drawn in the order
q, k, v, mask (as benchmark/benchmark_fa.py:100-112 of the reference draws
q, k, v, then the mask), so host oracles and the GPU see identical tensors.
Masks are additive: 0 = visible, -inf = blocked.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

NEG_INF = float("-inf")


@dataclass(frozen=True)
class Config:
    name: str
    B: int
    H: int
    Hk: int
    Sq: int
    Sk: int
    d: int
    dtype: torch.dtype
    mask_kind: str
    description: str

    @property
    def flops(self) -> float:
        """4·B·H·Sq·Sk·d, the reference's FLOP count (benchmark/benchmark_fa.py:135-137)."""
        return 4.0 * self.B * self.H * self.Sq * self.Sk * self.d

    @property
    def algorithmic_bytes(self) -> int:
        """Each of q, k, v, mask read once and o written once."""
        e = 2 if self.dtype in (torch.bfloat16, torch.float16) else 4
        q = self.B * self.H * self.Sq * self.d
        kv = self.B * self.Hk * self.Sk * self.d
        m = self.B * self.Sq * self.Sk
        return e * (2 * q + 2 * kv + m)


CONFIGS = {
    "cfg1": Config("cfg1", 1, 4, 4, 512, 512, 64, torch.float32, "causal",
                   "CPU plumbing: fp32, causal additive mask"),
    "cfg2": Config("cfg2", 4, 16, 16, 2048, 2048, 128, torch.bfloat16, "random10_diag",
                   "standard masked fwd, 10% i.i.d. -inf, diagonal visible"),
    "cfg3": Config("cfg3", 4, 16, 4, 2048, 2048, 128, torch.bfloat16, "random10_diag",
                   "GQA 16/4, same mask as cfg2"),
    "cfg4": Config("cfg4", 1, 16, 16, 128, 32768, 128, torch.bfloat16, "random10_first64",
                   "small-grid long-context split-KV, 10% -inf, keys 0..63 visible"),
    "cfg5": Config("cfg5", 2, 16, 4, 1000, 4099, 128, torch.bfloat16, "window_pad_random5",
                   "ragged: sliding window 1024 (bottom-right aligned) AND batch-1 keys >= 3799 "
                   "blocked AND 5% random"),
}


def make_mask(kind: str, B: int, Sq: int, Sk: int, g: torch.Generator) -> torch.Tensor:
    """fp32 additive mask [B,1,Sq,Sk] (cast to the config dtype by the caller)."""
    i = torch.arange(Sq).view(Sq, 1)
    j = torch.arange(Sk).view(1, Sk)
    if kind == "causal":
        vis = (j <= i).expand(Sq, Sk)
        blocked = (~vis).view(1, 1, Sq, Sk).expand(B, 1, Sq, Sk)
    elif kind == "random10_diag":
        blocked = torch.rand(B, 1, Sq, Sk, generator=g) < 0.10
        diag = (j == i).view(1, 1, Sq, Sk)
        blocked = blocked & ~diag
    elif kind == "random10_first64":
        blocked = torch.rand(B, 1, Sq, Sk, generator=g) < 0.10
        blocked[..., :64] = False
    elif kind == "window_pad_random5":
        off = Sk - Sq
        window = (j <= i + off) & (j > i + off - 1024)
        blocked = ~window.view(1, 1, Sq, Sk).expand(B, 1, Sq, Sk).clone()
        if B > 1:
            blocked[1, :, :, Sk - 300:] = True
        blocked = blocked | (torch.rand(B, 1, Sq, Sk, generator=g) < 0.05)
    elif kind == "zero":
        blocked = torch.zeros(B, 1, Sq, Sk, dtype=torch.bool)
    else:
        raise ValueError(f"unknown mask kind {kind!r}")
    return torch.zeros(B, 1, Sq, Sk).masked_fill(blocked, NEG_INF)


def make_inputs(cfg: Config, seed: int = 42, dtype: torch.dtype | None = None):
    """(q, k, v, mask) on CPU in ``dtype`` (default: the config's dtype)."""
    g = torch.Generator().manual_seed(seed)
    dt = dtype or cfg.dtype
    q = torch.randn(cfg.B, cfg.H, cfg.Sq, cfg.d, generator=g).to(dt)
    k = torch.randn(cfg.B, cfg.Hk, cfg.Sk, cfg.d, generator=g).to(dt)
    v = torch.randn(cfg.B, cfg.Hk, cfg.Sk, cfg.d, generator=g).to(dt)
    mask = make_mask(cfg.mask_kind, cfg.B, cfg.Sq, cfg.Sk, g).to(dt)
    return q, k, v, mask
