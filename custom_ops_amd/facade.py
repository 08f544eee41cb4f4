"""The package's front door: ``ops``, one object per process that hands out the
operator groups and the operators themselves.

Public surface (names, signatures and behaviour of the reference facade
``RecsysOps``, recsys.py:451-656, for the one group built here):

    ops.mha_fwd_with_mask(q, k, v, mask, backend=None)   recsys.py:641-656
    ops.is_available(group=None), ops.load_error(group=None), ops.groups
    ops.ensure_loaded(*groups), ops.load()
    ops.load_precompiled(group, library_path, metadata_path=None)
    ops.allow_jit / ops.configure(allow_jit=...) / ops.disable_jit()
    ops.<op name>  -> the dispatcher op, after its group is loaded

How it is organised here: the facade owns one ``_Slot`` per group. A slot
records the group's loader (created on first need) and where its library came
from: ``"tree"`` (development: the in-tree build, compiled by hipcc if it is
missing) or ``"artifact"`` (deployment: a sealed, validated export). The
policy is a single flag, ``allow_jit``; turning it off (explicitly, or by
loading an artifact) freezes the facade: from then on a slot is only ever
read, never loaded, and asking for an unloaded group raises
``CustomOpsError``.
"""
from __future__ import annotations

import os
import threading
from typing import Optional

import torch

from .loader import CustomOpsError, FAOps

# group name -> loader class; operator name -> group name
GROUP_LOADERS = {"fa": FAOps}
OP_GROUPS = {"mha_fwd_with_mask": "fa"}

_BACKENDS = ("auto", "cuda", "hip")


def resolve_backend(backend: Optional[str]) -> str:
    """The backend a call runs on: the argument, else ``CUSTOM_OPS_BACKEND``,
    else ``"auto"`` (the reference's order, recsys.py:140-158).

    Every accepted name means the same thing here, the HIP library (the device
    type is still called "cuda" on PyTorch-ROCm). ``"tilelang"`` is refused:
    there is no second backend and no silent fallback to one."""
    name = backend if backend is not None else os.environ.get("CUSTOM_OPS_BACKEND", "auto")
    name = str(name).strip().lower()
    if name == "tilelang":
        raise RuntimeError(
            "backend 'tilelang': the Tile-lang backend does not exist in this build; "
            "the HIP kernels for MI355X are the only backend (use backend='auto')")
    if name not in _BACKENDS:
        raise ValueError(f"backend {name!r} is not one of {list(_BACKENDS)} "
                         f"(argument or CUSTOM_OPS_BACKEND)")
    return name


def _as_flag(value) -> bool:
    if type(value) is not bool:
        raise TypeError(f"allow_jit must be a bool, not {type(value).__name__}")
    return value


class _Slot:
    """One op group as the facade sees it."""

    __slots__ = ("loader", "origin")

    def __init__(self) -> None:
        self.loader: Optional[FAOps] = None
        self.origin: Optional[str] = None     # None | "tree" | "artifact"

    @property
    def ready(self) -> bool:
        return self.loader is not None and self.loader.is_available()

    @property
    def state(self) -> str:
        if self.loader is None:
            return "not_loaded"
        return "loaded" if self.loader.is_available() else "failed"


class RecsysOps:
    """Facade over the operator groups (one group, ``fa``, in this build)."""

    def __init__(self, *, allow_jit: bool = True) -> None:
        self._mu = threading.RLock()
        self._slots = {name: _Slot() for name in GROUP_LOADERS}
        self._jit = _as_flag(allow_jit)

    # ── policy ──────────────────────────────────────────────────────────────
    @property
    def allow_jit(self) -> bool:
        """True: groups load lazily from the in-tree build. False: only groups
        loaded with ``load_precompiled`` are usable."""
        return self._jit

    @allow_jit.setter
    def allow_jit(self, value: bool) -> None:
        self.configure(allow_jit=value)

    def configure(self, *, allow_jit: bool) -> "RecsysOps":
        """Set the policy for this facade and every loader it holds; loads nothing."""
        flag = _as_flag(allow_jit)
        with self._mu:
            self._jit = flag
            for slot in self._slots.values():
                if slot.loader is not None:
                    slot.loader.configure(allow_jit=flag)
        return self

    def disable_jit(self) -> "RecsysOps":
        return self.configure(allow_jit=False)

    # ── groups ──────────────────────────────────────────────────────────────
    def _slot(self, group: str) -> _Slot:
        try:
            return self._slots[group]
        except (KeyError, TypeError):
            raise ValueError(f"unknown group {group!r}: this build provides "
                             f"{sorted(self._slots)}") from None

    def _acquire(self, group: str) -> FAOps:
        """The group's loader with its library loaded, loading it if the policy allows."""
        with self._mu:
            slot = self._slot(group)
            if slot.ready:
                return slot.loader
            if not self._jit:
                why = slot.loader.load_error() if slot.loader is not None else None
                raise CustomOpsError(
                    f"JIT is disabled and group {group!r} is not loaded: deploy it with "
                    f"ops.load_precompiled({group!r}, library_path, metadata_path=None)"
                    + (f"; its last load failed with: {why}" if why else ""))
            if slot.loader is None:
                slot.loader = GROUP_LOADERS[group](allow_jit=True)
            slot.loader.load()                  # raises CustomOpsError on failure
            slot.origin = "tree"
            return slot.loader

    def load_precompiled(self, group: str, library_path, metadata_path=None) -> "RecsysOps":
        """Validate and load a deployed library (sidecar defaults to
        ``<library_path>.json``). The facade stays in strict mode afterwards,
        whether or not the load succeeds."""
        with self._mu:
            slot = self._slot(group)
            self.configure(allow_jit=False)
            if slot.loader is None:
                slot.loader = GROUP_LOADERS[group](allow_jit=False)
            slot.loader.load_precompiled(library_path, metadata_path)
            slot.origin = "artifact"
        return self

    def ensure_loaded(self, *groups: str) -> "RecsysOps":
        """Load the named groups (all when none is named). Unknown names are
        rejected before anything loads."""
        with self._mu:
            for g in groups:
                self._slot(g)
            for g in groups or tuple(self._slots):
                self._acquire(g)
        return self

    def load(self) -> "RecsysOps":
        return self.ensure_loaded()

    @property
    def groups(self) -> dict:
        """``{group: "loaded" | "failed" | "not_loaded"}``."""
        with self._mu:
            return {name: slot.state for name, slot in self._slots.items()}

    def is_available(self, group: Optional[str] = None) -> bool:
        """Whether the named group (else the facade as a whole) can run.

        With ``allow_jit`` the question loads what it asks about; in strict mode
        it only reads the current state. Without a group it also needs a
        visible GPU, and in strict mode at least one deployed group."""
        with self._mu:
            if group is not None:
                slot = self._slot(group)
                if not self._jit:
                    return slot.ready
                try:
                    self._acquire(group)
                except CustomOpsError:
                    return False
                return True
            if not torch.cuda.is_available():
                return False
            if not self._jit:
                created = [s for s in self._slots.values() if s.loader is not None]
                return bool(created) and all(s.ready for s in created)
            try:
                self.ensure_loaded()
            except CustomOpsError:
                return False
            return True

    def load_error(self, group: Optional[str] = None) -> Optional[str]:
        """The last load error of the named group, else of the first failed
        one; never loads anything."""
        with self._mu:
            slots = [self._slot(group)] if group is not None else list(self._slots.values())
            for slot in slots:
                if slot.loader is not None and (group is not None or not slot.ready):
                    err = slot.loader.load_error()
                    if err or group is not None:
                        return err
        return None

    # ── operators ───────────────────────────────────────────────────────────
    def mha_fwd_with_mask(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          mask: torch.Tensor, backend: Optional[str] = None) -> torch.Tensor:
        """FlashAttention-2 forward with an additive fp16/bf16 mask (recsys.py:641-656).

        q [B,H,Sq,d], k/v [B,Hk,Sk,d] (H % Hk == 0), mask [B,1,>=Sq,>=Sk] with
        0 = visible, -inf = blocked, finite = bias. d in {64, 128}."""
        resolve_backend(backend)
        self._acquire(OP_GROUPS["mha_fwd_with_mask"])
        return torch.ops.recsys_ops.mha_fwd_with_mask(q, k, v, mask)

    def __getattr__(self, name: str):
        if name.startswith("_"):
            raise AttributeError(name)
        group = OP_GROUPS.get(name)
        if group is None:
            raise AttributeError(f"No op '{name}' in this build: it provides "
                                 f"{sorted(OP_GROUPS)} in groups {sorted(GROUP_LOADERS)}")
        self._acquire(group)
        return getattr(torch.ops.recsys_ops, name)

    def __repr__(self) -> str:
        origins = {n: s.origin for n, s in self._slots.items() if s.origin}
        return (f"RecsysOps(allow_jit={self._jit}, namespace='recsys_ops', backend='hip', "
                f"groups={self.groups}, origins={origins})")
