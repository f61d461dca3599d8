"""Model adapters for the invariance harness.  Only synthetic ones ship here: the reference's
adapters load published checkpoints (no network on this build's machines)."""

from .synthetic_vla import SyntheticVLAAdapter

ADAPTERS = {"synthetic_vla": SyntheticVLAAdapter}

__all__ = ["ADAPTERS", "SyntheticVLAAdapter"]
