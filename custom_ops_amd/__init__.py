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
from .loader import CustomOpsError, FAOps

__all__ = ["ops", "RecsysOps", "CustomOpsError", "FAOps", "mha_fwd_with_mask"]


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
    """Lazy facade over the op groups (reference ``RecsysOps``, recsys.py:451-640).
    Only the ``fa`` group exists here.

    Development (``allow_jit=True``, the default): a group loads on first use
    from the in-tree library (compiled with hipcc if missing). Deployment:
    ``load_precompiled('fa', path)`` validates and loads an exported library and
    switches the facade to strict mode, in which nothing is ever compiled and
    an unloaded group raises."""

    _GROUP_CLASSES = {"fa": FAOps}
    _OP_TO_GROUP = {"mha_fwd_with_mask": "fa"}

    def __init__(self, *, allow_jit: bool = True) -> None:
        self._lock = threading.RLock()
        self._groups: dict = {}     # group -> FAOps instance
        self._allow_jit = True
        self.configure(allow_jit=allow_jit)

    @property
    def allow_jit(self) -> bool:
        return self._allow_jit

    @allow_jit.setter
    def allow_jit(self, value: bool) -> None:
        self.configure(allow_jit=value)

    def configure(self, *, allow_jit: bool) -> "RecsysOps":
        """Policy for all current and future groups, without loading any."""
        if not isinstance(allow_jit, bool):
            raise TypeError("allow_jit must be a bool")
        with self._lock:
            self._allow_jit = allow_jit
            for inst in self._groups.values():
                inst.configure(allow_jit=allow_jit)
        return self

    def disable_jit(self) -> "RecsysOps":
        return self.configure(allow_jit=False)

    def _validate_group(self, name: str) -> None:
        if name not in self._GROUP_CLASSES:
            raise ValueError(f"unknown group {name!r}; available: {sorted(self._GROUP_CLASSES)}")

    def _group(self, name: str) -> FAOps:
        with self._lock:
            self._validate_group(name)
            if not self._allow_jit:
                inst = self._groups.get(name)
                if inst is None or not inst.is_available():
                    err = inst.load_error() if inst is not None else None
                    raise CustomOpsError(
                        f"JIT is disabled for group {name!r}; call "
                        f"load_precompiled({name!r}, library_path, metadata_path=None) first."
                        + (f" Previous error: {err}" if err else ""))
                return inst
            if name not in self._groups:
                self._groups[name] = self._GROUP_CLASSES[name](allow_jit=True)
            inst = self._groups[name]
            if not inst.is_available():
                inst.load()
            return inst

    def load_precompiled(self, group: str, library_path, metadata_path=None) -> "RecsysOps":
        """Validate and load an exported library; disables compiling for all groups."""
        with self._lock:
            self._validate_group(group)
            self.configure(allow_jit=False)
            if group not in self._groups:
                self._groups[group] = self._GROUP_CLASSES[group](allow_jit=False)
            self._groups[group].load_precompiled(library_path, metadata_path)
        return self

    def ensure_loaded(self, *names) -> "RecsysOps":
        targets = names or tuple(self._GROUP_CLASSES)
        with self._lock:
            for name in targets:
                self._validate_group(name)
            for name in targets:
                self._group(name)
        return self

    def load(self) -> "RecsysOps":
        return self.ensure_loaded()

    @property
    def groups(self) -> dict:
        with self._lock:
            return {g: ("loaded" if self._groups[g].is_available() else "failed")
                    if g in self._groups else "not_loaded" for g in self._GROUP_CLASSES}

    def is_available(self, group: str | None = None) -> bool:
        """True when the device is usable and the requested (or every) group loads.
        In strict mode a read-only query."""
        with self._lock:
            if group is not None:
                self._validate_group(group)
            if not torch.cuda.is_available():
                return False
            if not self._allow_jit:
                names = [group] if group else list(self._groups)
                return bool(names) and all(
                    n in self._groups and self._groups[n].is_available() for n in names)
            try:
                self.ensure_loaded(*([group] if group else []))
            except CustomOpsError:
                return False
            return True

    def load_error(self, group: str | None = None):
        with self._lock:
            if group is not None:
                self._validate_group(group)
                inst = self._groups.get(group)
                return inst.load_error() if inst is not None else None
            for inst in self._groups.values():
                if not inst.is_available():
                    return inst.load_error()
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
            f"(groups: {sorted(self._GROUP_CLASSES)})")

    def __repr__(self) -> str:
        return (f"RecsysOps(lazy, allow_jit={self.allow_jit}, namespace='recsys_ops', "
                f"backend='hip', groups={self.groups})")


ops = RecsysOps()


def mha_fwd_with_mask(q, k, v, mask, num_splits: int = 0):
    """Direct call into the HIP path; ``num_splits`` > 0 forces the split count."""
    return fa.mha_fwd_with_mask_hip(q, k, v, mask, num_splits=num_splits)
