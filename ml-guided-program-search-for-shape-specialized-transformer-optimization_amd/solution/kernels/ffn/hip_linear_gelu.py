"""Fused Linear + bias + exact GELU on gfx950 through the C ABI.

Counterpart of the reference's fused FFN input projection
(solution/kernels/ffn/triton_linear_exact_gelu.py): the same
``available / can_use / prevalidated`` triplet, the same ``(hidden, marker)``
return value and the same strictness (an unsupported launch raises
ValueError, a failed launch RuntimeError, no silent fallback).  The reference
kernel (:69-137) accumulates in fp32, adds the bias in fp32, applies
``0.5 v (1 + erf(v / sqrt(2)))`` and rounds once to fp16; this one does the
same for bf16 or fp16 operands and rounds once to the operand dtype.

The kernel is ``sah_linear`` (csrc/linear_gelu.hip) with one launch shape,
(block_m, block_n, block_k, num_warps, num_stages) = (256, 256, 64, 8, 2).
It needs in_features % 64 == 0 and out_features % 256 == 0.
"""

from __future__ import annotations

import torch

from ..hip._library import (
    SAH_ACTIVATION_GELU_EXACT,
    SAH_ACTIVATION_NONE,
    check_status,
    dtype_code,
    is_gfx950,
    library_available,
    load_library,
    stream_handle,
)

HIP_LINEAR_EXACT_GELU_BACKEND = "hip_linear_exact_gelu"
HIP_LINEAR_BACKEND = "hip_linear"

DEFAULT_BLOCK_M = 256
DEFAULT_BLOCK_N = 256
DEFAULT_BLOCK_K = 64
DEFAULT_NUM_WARPS = 8
DEFAULT_NUM_STAGES = 2
IN_FEATURES_MULTIPLE = 64
OUT_FEATURES_MULTIPLE = 256
_SUPPORTED_DTYPES = frozenset({torch.bfloat16, torch.float16})


def launch_config_is_valid(
    block_m: int, block_n: int, block_k: int, num_warps: int, num_stages: int
) -> bool:
    """The launch the gfx950 kernel implements (the C library's own table)."""

    values = (block_m, block_n, block_k, num_warps, num_stages)
    if any(isinstance(value, bool) or not isinstance(value, int) for value in values):
        return False
    if library_available():
        return bool(load_library().sah_linear_launch_supported(*values))
    return values == (
        DEFAULT_BLOCK_M,
        DEFAULT_BLOCK_N,
        DEFAULT_BLOCK_K,
        DEFAULT_NUM_WARPS,
        DEFAULT_NUM_STAGES,
    )


def _validate_launch_config(
    block_m: int, block_n: int, block_k: int, num_warps: int, num_stages: int
) -> None:
    if not launch_config_is_valid(block_m, block_n, block_k, num_warps, num_stages):
        raise ValueError("unsupported HIP Linear + Exact-GELU launch configuration")


def supported_features(in_features: int, out_features: int) -> bool:
    """Feature sizes with a kernel instantiation."""

    return (
        in_features > 0
        and out_features > 0
        and in_features % IN_FEATURES_MULTIPLE == 0
        and out_features % OUT_FEATURES_MULTIPLE == 0
    )


def hip_linear_exact_gelu_available() -> bool:
    """Whether the gfx950 library loads in this process."""

    return library_available()


def can_use_hip_linear_exact_gelu(
    value: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None
) -> bool:
    """Whether the fused kernel implements these Linear operands
    (the reference's eligibility rules, triton_linear_exact_gelu.py:145-178,
    with this kernel's dtypes and feature sizes)."""

    tensors = [value, weight] + ([] if bias is None else [bias])
    if not all(isinstance(item, torch.Tensor) for item in tensors):
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return False
    if value.device.type != "cuda" or any(t.device != value.device for t in tensors):
        return False
    if value.ndim < 2 or weight.ndim != 2 or (bias is not None and bias.ndim != 1):
        return False
    if value.numel() == 0 or value.shape[-1] != weight.shape[1]:
        return False
    if bias is not None and bias.shape[0] != weight.shape[0]:
        return False
    if not supported_features(weight.shape[1], weight.shape[0]):
        return False
    if value.dtype not in _SUPPORTED_DTYPES or any(t.dtype != value.dtype for t in tensors):
        return False
    if not all(t.is_contiguous() for t in tensors):
        return False
    if value.data_ptr() % 16 or weight.data_ptr() % 16 or (bias is not None and bias.data_ptr() % 8):
        return False
    if not library_available():
        return False
    return is_gfx950(value.device)


def _launch(
    value: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    activation: int,
    launch: tuple[int, int, int, int, int],
) -> torch.Tensor:
    in_features = value.shape[-1]
    out_features = weight.shape[0]
    rows = value.numel() // in_features
    output = torch.empty((*value.shape[:-1], out_features), device=value.device, dtype=value.dtype)
    status = load_library().sah_linear(
        value.data_ptr(),
        weight.data_ptr(),
        None if bias is None else bias.data_ptr(),
        output.data_ptr(),
        rows,
        in_features,
        out_features,
        in_features,
        out_features,
        dtype_code(value.dtype),
        activation,
        *launch,
        stream_handle(value.device),
    )
    check_status(status, "HIP Linear + Exact-GELU execution")
    return output


def prevalidated_hip_linear_exact_gelu(
    value: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    *,
    block_m: int = DEFAULT_BLOCK_M,
    block_n: int = DEFAULT_BLOCK_N,
    block_k: int = DEFAULT_BLOCK_K,
    num_warps: int = DEFAULT_NUM_WARPS,
    num_stages: int = DEFAULT_NUM_STAGES,
) -> tuple[torch.Tensor, str]:
    """GELU(value @ weight.T + bias) after the caller established eligibility
    (reference: prevalidated_triton_linear_exact_gelu, :182-234)."""

    _validate_launch_config(block_m, block_n, block_k, num_warps, num_stages)
    if not can_use_hip_linear_exact_gelu(value, weight, bias):
        raise RuntimeError("HIP Linear + Exact-GELU inputs are ineligible for the gfx950 kernel")
    hidden = _launch(
        value, weight, bias, SAH_ACTIVATION_GELU_EXACT, (block_m, block_n, block_k, num_warps, num_stages)
    )
    return hidden, HIP_LINEAR_EXACT_GELU_BACKEND


def prevalidated_hip_linear(
    value: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    block_m: int = DEFAULT_BLOCK_M,
    block_n: int = DEFAULT_BLOCK_N,
    block_k: int = DEFAULT_BLOCK_K,
    num_warps: int = DEFAULT_NUM_WARPS,
    num_stages: int = DEFAULT_NUM_STAGES,
) -> tuple[torch.Tensor, str]:
    """value @ weight.T + bias with the same kernel and no activation."""

    _validate_launch_config(block_m, block_n, block_k, num_warps, num_stages)
    if not can_use_hip_linear_exact_gelu(value, weight, bias):
        raise RuntimeError("HIP Linear inputs are ineligible for the gfx950 kernel")
    output = _launch(
        value, weight, bias, SAH_ACTIVATION_NONE, (block_m, block_n, block_k, num_warps, num_stages)
    )
    return output, HIP_LINEAR_BACKEND


__all__ = [
    "DEFAULT_BLOCK_K",
    "DEFAULT_BLOCK_M",
    "DEFAULT_BLOCK_N",
    "DEFAULT_NUM_STAGES",
    "DEFAULT_NUM_WARPS",
    "HIP_LINEAR_BACKEND",
    "HIP_LINEAR_EXACT_GELU_BACKEND",
    "can_use_hip_linear_exact_gelu",
    "hip_linear_exact_gelu_available",
    "launch_config_is_valid",
    "prevalidated_hip_linear",
    "prevalidated_hip_linear_exact_gelu",
    "supported_features",
]
