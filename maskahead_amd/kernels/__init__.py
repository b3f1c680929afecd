"""gfx950 kernel ops of the KV read/keep path (the reference's maskahead.kernels)."""

from .ops import (
    KernelUnavailableError,
    dense_packed_attention,
    gather_packed_kv,
    hip_available,
    quantize_key_groups_into,
    quantize_values_into,
    selector_topk,
)
from .select import prefix_scores_topk, topk_ascending
from .splitk import Prefix, dequantize_prefix, prefix_scores, splitk_attention
from .step0 import Step0Buffers, step0_select

__all__ = [
    "KernelUnavailableError",
    "Prefix",
    "dense_packed_attention",
    "dequantize_prefix",
    "gather_packed_kv",
    "hip_available",
    "prefix_scores",
    "prefix_scores_topk",
    "quantize_key_groups_into",
    "quantize_values_into",
    "selector_topk",
    "splitk_attention",
    "Step0Buffers",
    "step0_select",
    "topk_ascending",
]
