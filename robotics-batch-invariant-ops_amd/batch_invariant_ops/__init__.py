"""batch_invariant_ops for AMD Instinct MI355X: same public API as the reference package
(yiannisha/robotics-batch-invariant-ops, batch_invariant_ops/__init__.py:1-49), backed by the
hand-written gfx950 HIP kernels of libbiops.so."""

from .batch_invariant_ops import (
    set_batch_invariant_mode,
    is_batch_invariant_mode_enabled,
    disable_batch_invariant_mode,
    enable_batch_invariant_mode,
    matmul_persistent,
    linear_batch_invariant,
    bmm_persistent,
    conv1d_batch_invariant,
    conv2d_batch_invariant,
    conv3d_batch_invariant,
    conv_transpose2d_batch_invariant,
    conv_transpose3d_batch_invariant,
    scaled_dot_product_attention_batch_invariant,
    varlen_scaled_dot_product_attention_batch_invariant,
    linalg_vector_norm_batch_invariant,
    softmax,
    log_softmax,
    mean_dim,
    get_batch_invariant_attention_block_size,
    AttentionBlockSize,
)
from .moe import deterministic_token_choice_moe

__version__ = "0.2.0"

__all__ = [
    "set_batch_invariant_mode",
    "is_batch_invariant_mode_enabled",
    "disable_batch_invariant_mode",
    "enable_batch_invariant_mode",
    "matmul_persistent",
    "linear_batch_invariant",
    "bmm_persistent",
    "conv1d_batch_invariant",
    "conv2d_batch_invariant",
    "conv3d_batch_invariant",
    "conv_transpose2d_batch_invariant",
    "conv_transpose3d_batch_invariant",
    "scaled_dot_product_attention_batch_invariant",
    "varlen_scaled_dot_product_attention_batch_invariant",
    "linalg_vector_norm_batch_invariant",
    "softmax",
    "log_softmax",
    "mean_dim",
    "get_batch_invariant_attention_block_size",
    "AttentionBlockSize",
    "deterministic_token_choice_moe",
]
