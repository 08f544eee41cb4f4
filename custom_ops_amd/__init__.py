"""custom_ops_amd — MI355X-native ``mha_fwd_with_mask`` (masked FlashAttention-2 forward).

Drop-in for the reference facade (Defyli/custom_ops ``recsys.py``), also
importable under the reference's own package name::

    from custom_ops import ops                          # or: from custom_ops_amd import ops
    out = ops.mha_fwd_with_mask(q, k, v, mask)          # recsys.py:641-656
    ops.is_available(); ops.load_error(); ops.groups    # recsys.py:542-581

and for the dispatcher op ``torch.ops.recsys_ops.mha_fwd_with_mask`` with the
reference's schema (csrc/fa/fa_bindings.cpp:37-43). The compute runs in the
hand-written HIP library ``libmi355_fa.so`` (gfx950); there is no fallback: if
the library is missing, calls raise ``RuntimeError``.
"""
from __future__ import annotations

from . import _lib, fa
from .facade import RecsysOps, resolve_backend
from ._lib import Variant
from .loader import CustomOpsError, FAOps

__all__ = ["ops", "RecsysOps", "CustomOpsError", "FAOps", "Variant", "mha_fwd_with_mask"]

_resolve_backend = resolve_backend

ops = RecsysOps()


def mha_fwd_with_mask(q, k, v, mask, num_splits: int = 0, variant=None):
    """Direct call into the HIP path; ``num_splits`` > 0 forces the split count
    and ``variant`` (a ``custom_ops_amd.Variant``) selects kernel variants for
    tests and tuning."""
    return fa.mha_fwd_with_mask_hip(q, k, v, mask, num_splits=num_splits, variant=variant)
