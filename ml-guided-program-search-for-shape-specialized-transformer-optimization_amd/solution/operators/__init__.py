"""Portable PyTorch operators of the plan API (the reference-order program)."""

from .attention.sdpa import can_use_causal_sdpa, causal_sdpa, reference_causal_attention
from .norm.residual_add import can_use_residual_add, residual_add
from .projection.qkv_layout import can_split_qkv, split_qkv

__all__ = [
    "can_split_qkv",
    "can_use_causal_sdpa",
    "can_use_residual_add",
    "causal_sdpa",
    "reference_causal_attention",
    "residual_add",
    "split_qkv",
]
