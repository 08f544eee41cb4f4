"""custom_ops_amd — MI355X-native ``mha_fwd_with_mask`` (masked FlashAttention-2 forward).

Drop-in for the reference facade (Defyli/custom_ops ``recsys.py``):

    from custom_ops_amd import ops
    out = ops.mha_fwd_with_mask(q, k, v, mask)          # recsys.py:641-656
    ops.is_available(); ops.load_error(); ops.groups    # recsys.py:542-581

and for the dispatcher op ``torch.ops.recsys_ops.mha_fwd_with_mask`` with the
reference's schema (csrc/fa/fa_bindings.cpp:37-43). The compute runs in the
hand-written HIP library ``libmi355_fa.so`` (gfx950); there is no fallback: if
the library is missing, calls raise ``RuntimeError``.
"""
from __future__ import annotations

import os
import threading

import torch

from . import _lib, fa

__all__ = ["ops", "RecsysOps", "CustomOpsError", "mha_fwd_with_mask"]


class CustomOpsError(RuntimeError):
    """Load/dispatch failure (the reference raises the same class name, __init__.py)."""


def _resolve_backend(backend):
    """Explicit argument > env CUSTOM_OPS_BACKEND > "auto" (recsys.py:140-158).

    "auto", "cuda" and "hip" all select the HIP library (on PyTorch-ROCm the
    device type is still called "cuda"). "tilelang" is not provided: this
    package has exactly one backend and never falls back to another."""
    if backend is None:
        backend = os.environ.get("CUSTOM_OPS_BACKEND", "auto")
    backend = str(backend).lower()
    if backend not in ("auto", "cuda", "hip", "tilelang"):
        raise ValueError(
            f"backend must be 'auto' | 'cuda' | 'hip', got {backend!r} "
            f"(or set CUSTOM_OPS_BACKEND env)")
    if backend == "tilelang":
        raise RuntimeError("the Tile-lang backend is not part of custom_ops_amd; "
                           "use backend='auto' (HIP kernels for MI355X)")
    return backend


class RecsysOps:
    """Lazy facade over the op groups. Only the ``fa`` group exists here."""

    _GROUPS = ("fa",)
    _OP_TO_GROUP = {"mha_fwd_with_mask": "fa"}

    def __init__(self) -> None:
        self._lock = threading.RLock()
        self._state = {}     # group -> "loaded" | "failed"
        self._errors = {}

    def _validate_group(self, name: str) -> None:
        if name not in self._GROUPS:
            raise ValueError(f"unknown group {name!r}; available: {sorted(self._GROUPS)}")

    def _group(self, name: str) -> None:
        with self._lock:
            self._validate_group(name)
            if self._state.get(name) == "loaded":
                return
            try:
                _lib.load()
                fa.register()
            except Exception as e:  # keep the reason, fail loudly at use
                self._state[name] = "failed"
                self._errors[name] = str(e)
                raise CustomOpsError(f"group {name!r} failed to load: {e}") from e
            self._state[name] = "loaded"
            self._errors.pop(name, None)

    def ensure_loaded(self, *names) -> "RecsysOps":
        for name in (names or self._GROUPS):
            self._group(name)
        return self

    def load(self) -> "RecsysOps":
        return self.ensure_loaded()

    @property
    def groups(self) -> dict:
        with self._lock:
            return {g: self._state.get(g, "not_loaded") for g in self._GROUPS}

    def is_available(self, group: str | None = None) -> bool:
        """True when the device is usable and the requested (or every) group loads."""
        if group is not None:
            self._validate_group(group)
        if not torch.cuda.is_available():
            return False
        try:
            self.ensure_loaded(*( [group] if group else []))
        except CustomOpsError:
            return False
        return True

    def load_error(self, group: str | None = None):
        with self._lock:
            if group is not None:
                self._validate_group(group)
                return self._errors.get(group)
            for g in self._GROUPS:
                if g in self._errors:
                    return self._errors[g]
        return None

    def mha_fwd_with_mask(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          mask: torch.Tensor, backend: str | None = None) -> torch.Tensor:
        """FlashAttention-2 forward with an additive fp16/bf16 mask (recsys.py:641-656).

        q [B,H,Sq,d], k/v [B,Hk,Sk,d] (H % Hk == 0), mask [B,1,>=Sq,>=Sk] with
        0 = visible, -inf = blocked, finite = bias. d in {64, 128}."""
        _resolve_backend(backend)
        self._group("fa")
        return torch.ops.recsys_ops.mha_fwd_with_mask(q, k, v, mask)

    def __getattr__(self, name: str):
        if name.startswith("_"):
            raise AttributeError(name)
        raise AttributeError(
            f"No op '{name}' in recsys_ops. Available ops: {sorted(self._OP_TO_GROUP)} "
            f"(groups: {sorted(self._GROUPS)})")

    def __repr__(self) -> str:
        return f"RecsysOps(namespace='recsys_ops', backend='hip', groups={self.groups})"


ops = RecsysOps()


def mha_fwd_with_mask(q, k, v, mask, num_splits: int = 0):
    """Direct call into the HIP path; ``num_splits`` > 0 forces the split count."""
    return fa.mha_fwd_with_mask_hip(q, k, v, mask, num_splits=num_splits)
