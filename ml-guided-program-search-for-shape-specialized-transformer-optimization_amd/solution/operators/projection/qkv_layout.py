"""Zero-copy split of a packed QKV projection into [B, H, S, Dh] views.

Same contract as the reference's solution/operators/projection/qkv_layout.py:
22-50: ``[B, S, 3D]`` with unit last stride becomes three views with strides
``(S*3D, Dh, 3D, 1)``; ``contiguous=True`` materializes them.  The gfx950
attention kernel reads these strided views directly (16-byte rows).
"""

from __future__ import annotations

import torch


def can_split_qkv(packed_qkv: torch.Tensor, num_heads: int) -> bool:
    if packed_qkv.ndim != 3 or num_heads <= 0 or packed_qkv.stride(-1) != 1:
        return False
    width = packed_qkv.shape[-1]
    if width <= 0 or width % 3:
        return False
    return (width // 3) % num_heads == 0


def split_qkv(
    packed_qkv: torch.Tensor,
    num_heads: int,
    *,
    contiguous: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    if not can_split_qkv(packed_qkv, num_heads):
        raise ValueError("packed QKV shape is incompatible with num_heads")
    model_width = packed_qkv.shape[-1] // 3
    heads = packed_qkv.view(*packed_qkv.shape[:-1], 3, num_heads, model_width // num_heads)
    query, key, value = (heads.select(-3, index).transpose(1, 2) for index in range(3))
    if contiguous:
        return query.contiguous(), key.contiguous(), value.contiguous()
    return query, key, value


__all__ = ["can_split_qkv", "split_qkv"]
