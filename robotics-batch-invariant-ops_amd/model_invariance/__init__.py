"""Model-level batch-invariance investigation (reference scripts/model_invariance/__init__.py)."""

from .harness import (
    DEFAULT_BATCH_SIZES,
    ModelAdapter,
    TensorDifference,
    compare_outputs,
    run_investigation,
    seed_everything,
)

__all__ = [
    "DEFAULT_BATCH_SIZES",
    "ModelAdapter",
    "TensorDifference",
    "compare_outputs",
    "run_investigation",
    "seed_everything",
]
