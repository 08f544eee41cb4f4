"""``custom_ops`` — the reference's import name for this package.

Code written against Defyli/custom_ops imports ``from custom_ops import ops``
(examples/basic_usage.py:24) and ``from custom_ops.recsys import ...``; both
resolve here to the MI355X build in ``custom_ops_amd``, so such code runs
unchanged. Only the ``fa`` group (``mha_fwd_with_mask``) exists in this build.
"""
from custom_ops_amd import CustomOpsError, FAOps, RecsysOps, ops

__all__ = ["ops", "RecsysOps", "FAOps", "CustomOpsError"]
