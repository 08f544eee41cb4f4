"""Committed golden fixtures for mha_fwd_with_mask (see make_golden.py)."""
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE_FILE = os.path.join(HERE, "fa_fixtures.npz")


@dataclass
class Fixture:
    name: str
    dtype: str            # "bf16" | "fp16"
    q: np.ndarray         # uint16 bit patterns
    k: np.ndarray
    v: np.ndarray
    mask: np.ndarray
    sq: int
    sk: int
    expected: np.ndarray  # float32, fp64 closed form on the dtype-exact inputs
    masked_rows: list

    def to_f32(self, a):
        if self.dtype == "bf16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        return a.view(np.float16).astype(np.float32)

    def tensors_f32(self):
        return tuple(self.to_f32(a) for a in (self.q, self.k, self.v, self.mask))

    def tensors_torch(self):
        import torch
        dt = torch.bfloat16 if self.dtype == "bf16" else torch.float16
        return tuple(torch.from_numpy(a.view(np.int16).copy()).view(dt)
                     for a in (self.q, self.k, self.v, self.mask))


def load_fixtures():
    data = np.load(FIXTURE_FILE, allow_pickle=False)
    names = [str(n) for n in data["names"]]
    out = []
    for n in names:
        meta = data[f"{n}__meta"]
        out.append(Fixture(
            name=n, dtype="bf16" if int(meta[0]) == 1 else "fp16",
            q=data[f"{n}__q"], k=data[f"{n}__k"], v=data[f"{n}__v"], mask=data[f"{n}__mask"],
            sq=int(meta[1]), sk=int(meta[2]), expected=data[f"{n}__expected"],
            masked_rows=[int(r) for r in data[f"{n}__masked_rows"]]))
    return out
