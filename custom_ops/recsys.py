"""``custom_ops.recsys`` — the reference module that defines the facade
(recsys.py), for imports such as ``from custom_ops.recsys import FAOps, RecsysOps``."""
from custom_ops_amd import FAOps, RecsysOps, ops

__all__ = ["ops", "RecsysOps", "FAOps"]
