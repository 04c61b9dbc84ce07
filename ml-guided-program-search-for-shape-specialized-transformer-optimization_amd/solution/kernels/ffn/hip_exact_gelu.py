"""Elementwise exact GELU on gfx950 through the C ABI.

Counterpart of the reference's Exact-GELU primitive
(solution/kernels/ffn/triton_exact_gelu.py): the same
``available / can_use / prevalidated / checked`` functions, the same
``(hidden, marker)`` return value and the same strictness (ValueError for an
unsupported launch, RuntimeError for ineligible inputs or a failed launch, no
silent fallback).  The reference evaluates GELU in fp32 and casts once to the
output dtype (:50-68); this kernel does the same for bf16/fp16 tensors, with
the output dtype equal to the input's.  ``out`` may be the input itself (the
FFN path applies the activation in place on the projection it just made).

Launch: ``block_size`` elements per workgroup of ``num_warps`` wavefronts,
block_size = 512 x num_warps x {1, 2, 4, 8} (16-byte chunks per thread).
"""

from __future__ import annotations

import torch

from ..hip._library import (
    check_status,
    dtype_code,
    is_gfx950,
    library_available,
    load_library,
    stream_handle,
)

HIP_EXACT_GELU_BACKEND = "hip_exact_gelu"
DEFAULT_BLOCK_SIZE = 4096
DEFAULT_NUM_WARPS = 4
SUPPORTED_NUM_WARPS = frozenset({1, 2, 4, 8})
_SUPPORTED_DTYPES = frozenset({torch.bfloat16, torch.float16})


def launch_config_is_valid(block_size: int, num_warps: int) -> bool:
    """The launches the kernel implements (the C library's own rule)."""

    values = (block_size, num_warps)
    if any(isinstance(value, bool) or not isinstance(value, int) for value in values):
        return False
    if num_warps not in SUPPORTED_NUM_WARPS or block_size <= 0:
        return False
    per_pass = num_warps * 64 * 8
    return block_size % per_pass == 0 and block_size // per_pass in {1, 2, 4, 8}


def _validate_launch_config(block_size: int, num_warps: int) -> None:
    if not launch_config_is_valid(block_size, num_warps):
        raise ValueError("unsupported HIP Exact-GELU launch configuration")


def hip_exact_gelu_available() -> bool:
    """Whether the gfx950 library loads in this process."""

    return library_available()


def can_use_hip_exact_gelu(value: torch.Tensor, *, output_dtype: torch.dtype | None = None) -> bool:
    """Whether the kernel accepts this tensor (reference rules,
    triton_exact_gelu.py:71-90, with this kernel's dtypes)."""

    if not isinstance(value, torch.Tensor):
        return False
    if torch.is_grad_enabled() and value.requires_grad:
        return False
    if value.device.type != "cuda" or value.dtype not in _SUPPORTED_DTYPES:
        return False
    if output_dtype is not None and output_dtype != value.dtype:
        return False
    if not value.is_contiguous() or value.numel() == 0 or value.data_ptr() % 16:
        return False
    if not library_available():
        return False
    return is_gfx950(value.device)


def prevalidated_hip_exact_gelu(
    value: torch.Tensor,
    *,
    output_dtype: torch.dtype | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
    num_warps: int = DEFAULT_NUM_WARPS,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, str]:
    """GELU(value) after the caller established eligibility
    (reference: prevalidated_triton_exact_gelu, :93-118)."""

    _validate_launch_config(block_size, num_warps)
    if not can_use_hip_exact_gelu(value, output_dtype=output_dtype):
        raise RuntimeError("HIP Exact-GELU inputs are ineligible for the gfx950 kernel")
    if out is None:
        out = torch.empty_like(value)
    elif (
        out.shape != value.shape
        or out.dtype != value.dtype
        or out.device != value.device
        or not out.is_contiguous()
        or out.data_ptr() % 16
    ):
        raise RuntimeError("HIP Exact-GELU output buffer does not match the input")
    status = load_library().sah_gelu(
        value.data_ptr(),
        out.data_ptr(),
        value.numel(),
        dtype_code(value.dtype),
        block_size,
        num_warps,
        stream_handle(value.device),
    )
    check_status(status, "HIP Exact-GELU execution")
    return out, HIP_EXACT_GELU_BACKEND


def hip_exact_gelu(
    value: torch.Tensor,
    *,
    output_dtype: torch.dtype | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
    num_warps: int = DEFAULT_NUM_WARPS,
) -> tuple[torch.Tensor, str]:
    """Checked entry (reference: triton_exact_gelu, :121-140)."""

    _validate_launch_config(block_size, num_warps)
    if not can_use_hip_exact_gelu(value, output_dtype=output_dtype):
        raise RuntimeError("HIP Exact-GELU is ineligible for the requested input")
    return prevalidated_hip_exact_gelu(
        value, output_dtype=output_dtype, block_size=block_size, num_warps=num_warps
    )


__all__ = [
    "DEFAULT_BLOCK_SIZE",
    "DEFAULT_NUM_WARPS",
    "HIP_EXACT_GELU_BACKEND",
    "can_use_hip_exact_gelu",
    "hip_exact_gelu",
    "hip_exact_gelu_available",
    "launch_config_is_valid",
    "prevalidated_hip_exact_gelu",
]
