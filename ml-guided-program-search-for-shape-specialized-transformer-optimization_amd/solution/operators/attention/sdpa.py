"""Portable causal attention operators (PyTorch).

* ``reference_causal_attention`` keeps the official operation order (QK^T,
  scale, -inf causal and key masks, softmax in fp32, cast, PV) while bounding
  temporaries to ``[B, H, query_block, S]`` -- the contract of the reference's
  solution/operators/attention/sdpa.py:116-170.
* ``causal_sdpa`` is torch's scaled_dot_product_attention with the implicit
  causal bias (reference :76-113); like the reference it refuses bf16, whose
  different rounding boundaries can break the elementwise comparator.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_REFERENCE_QUERY_BLOCK = 128


def _attention_inputs_are_legal(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_token_mask: torch.Tensor | None,
    *,
    causal: bool,
) -> bool:
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        return False
    if query.device != key.device or query.device != value.device:
        return False
    if query.dtype not in _SUPPORTED_DTYPES:
        return False
    if key.dtype != query.dtype or value.dtype != query.dtype:
        return False
    if query.shape[:-1] != key.shape[:-1] or query.shape[:3] != value.shape[:3]:
        return False
    if query.shape[-1] != key.shape[-1]:
        return False
    if query.shape[-2] <= 0 or key.shape[-2] <= 0:
        return False
    if causal and query.shape[-2] != key.shape[-2]:
        return False
    return valid_token_mask is None or bool(
        valid_token_mask.device == query.device
        and valid_token_mask.dtype == torch.bool
        and valid_token_mask.ndim == 2
        and valid_token_mask.shape == (query.shape[0], key.shape[-2])
    )


def can_use_causal_sdpa(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_token_mask: torch.Tensor | None = None,
    *,
    causal: bool = True,
) -> bool:
    return bool(
        query.dtype != torch.bfloat16
        and _attention_inputs_are_legal(query, key, value, valid_token_mask, causal=causal)
    )


def causal_sdpa(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_token_mask: torch.Tensor | None = None,
    *,
    scale: float | None = None,
    causal: bool = True,
) -> torch.Tensor:
    if not can_use_causal_sdpa(query, key, value, valid_token_mask, causal=causal):
        raise ValueError("attention tensors are incompatible with causal SDPA")
    mask = None if valid_token_mask is None else valid_token_mask[:, None, None, :]
    return F.scaled_dot_product_attention(
        query, key, value, attn_mask=mask, dropout_p=0.0, is_causal=causal, scale=scale
    )


def reference_causal_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_token_mask: torch.Tensor | None = None,
    *,
    scale: float | None = None,
    causal: bool = True,
    query_block_size: int = _REFERENCE_QUERY_BLOCK,
) -> torch.Tensor:
    if (
        isinstance(query_block_size, bool)
        or not isinstance(query_block_size, int)
        or query_block_size <= 0
    ):
        raise ValueError("query_block_size must be a positive integer")
    if not _attention_inputs_are_legal(query, key, value, valid_token_mask, causal=causal):
        raise ValueError("attention tensors are incompatible with the safe path")
    effective_scale = query.shape[-1] ** -0.5 if scale is None else scale
    seq = query.shape[-2]
    key_positions = torch.arange(seq, device=query.device)
    # Batched GEMMs get dense operands: on ROCm, bf16 batched products with a
    # transposed or strided right operand are avoided entirely.
    key_t = key.transpose(-2, -1).contiguous()
    if query.device.type == "cuda":
        query = query.contiguous()
        value = value.contiguous()
    invalid_keys = None if valid_token_mask is None else (~valid_token_mask)[:, None, None, :]
    blocks = []
    for start in range(0, seq, query_block_size):
        stop = min(start + query_block_size, seq)
        scores = torch.matmul(query[..., start:stop, :], key_t)
        scores.mul_(effective_scale)
        if causal:
            rows = torch.arange(start, stop, device=query.device)
            scores.masked_fill_(key_positions[None, :] > rows[:, None], float("-inf"))
        if invalid_keys is not None:
            scores.masked_fill_(invalid_keys, float("-inf"))
        probabilities = torch.softmax(scores.float(), dim=-1).to(query.dtype)
        blocks.append(torch.matmul(probabilities, value))
    return torch.cat(blocks, dim=-2)


__all__ = ["can_use_causal_sdpa", "causal_sdpa", "reference_causal_attention"]
