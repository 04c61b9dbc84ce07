"""Linear + residual add + LayerNorm boundary on gfx950 through the C ABI.

Counterpart of the reference's fused linear boundary
(solution/kernels/boundary/triton_linear_residual_norm.py:1-245): the same
``available / can_use / strict`` functions, the same
``(source, weight, linear_bias, value, layer_norm, *, final_boundary,
block_rows, num_warps)`` call and ``(residual, normalized, marker)`` return
value, the same strictness (ineligible inputs raise RuntimeError "...
ineligible", a failed launch RuntimeError "... execution failed").  The
reference kernel (:34-109) multiplies a row block by the square projection
weight, adds the bias, rounds the update to its fp16 branch dtype, adds it to
the fp32 residual stream and normalizes, without writing the update.  This
one (``sah_linear_residual_norm``, csrc/linear_norm.hip) does the same on a
bf16 or fp16 stream: the update is rounded to the stream dtype, the residual
and the normalized rows are the stream dtype (there is no separate fp32
final-boundary output: the stream is the model dtype), and the projection may
be rectangular, so it serves both the attention output projection
(in = width) and the FFN output projection (in = ffn_dim).

Domain: width (d_model) 512 or 1024, in_features a multiple of 64; launch
block_rows = 65536 / width whole rows per workgroup, num_warps = 8 (the
reference's block_rows / num_warps launch fields, solution/config.py:327-355).
"""

from __future__ import annotations

import torch
from torch import nn

from ..hip._library import (
    SAH_NORM_LAYER,
    check_status,
    dtype_code,
    is_gfx950,
    library_available,
    load_library,
    stream_handle,
)

HIP_LINEAR_RESIDUAL_NORM_BACKEND = "hip_linear_residual_norm"
SUPPORTED_WIDTHS = frozenset({512, 1024})
IN_FEATURES_MULTIPLE = 64
NUM_WARPS = 8
_SUPPORTED_DTYPES = frozenset({torch.bfloat16, torch.float16})


def block_rows_for(width: int) -> int:
    """The implemented rows per workgroup for ``width`` (65536 / width)."""

    return 65536 // width


def launch_config_is_valid(width: int, block_rows: int, num_warps: int) -> bool:
    """The launch the gfx950 kernel implements for this width (the C
    library's own table)."""

    values = (width, block_rows, num_warps)
    if any(isinstance(value, bool) or not isinstance(value, int) for value in values):
        return False
    if library_available():
        return bool(load_library().sah_linear_residual_norm_launch_supported(*values))
    return width in SUPPORTED_WIDTHS and block_rows == block_rows_for(width) and num_warps == NUM_WARPS


def supported_width(width: int, in_features: int) -> bool:
    """Shapes with a kernel instantiation."""

    return width in SUPPORTED_WIDTHS and in_features > 0 and in_features % IN_FEATURES_MULTIPLE == 0


def hip_linear_residual_norm_available() -> bool:
    """Whether the gfx950 library loads in this process."""

    return library_available()


def can_use_hip_linear_residual_norm(
    source: torch.Tensor,
    weight: torch.Tensor,
    linear_bias: torch.Tensor | None,
    value: torch.Tensor,
    layer_norm: nn.LayerNorm,
    *,
    block_rows: int,
    num_warps: int,
) -> bool:
    """The reference's eligibility rules (triton_linear_residual_norm.py:124-194)
    with this kernel's dtypes and shapes; never raises."""

    tensors = [source, weight, value] + ([] if linear_bias is None else [linear_bias])
    if not all(isinstance(item, torch.Tensor) for item in tensors):
        return False
    if not isinstance(layer_norm, nn.LayerNorm) or torch.is_grad_enabled():
        return False
    if source.ndim != 3 or value.ndim != 3 or weight.ndim != 2:
        return False
    width, in_features = weight.shape
    if not supported_width(width, in_features) or not launch_config_is_valid(width, block_rows, num_warps):
        return False
    if tuple(source.shape) != (*value.shape[:2], in_features) or value.shape[-1] != width:
        return False
    if linear_bias is not None and linear_bias.shape != (width,):
        return False
    if tuple(layer_norm.normalized_shape) != (width,):
        return False
    params = [t for t in (layer_norm.weight, layer_norm.bias) if t is not None]
    if value.dtype not in _SUPPORTED_DTYPES or any(t.dtype != value.dtype for t in tensors + params):
        return False
    if source.device.type != "cuda" or any(t.device != source.device for t in tensors + params):
        return False
    # rows of the source: unit element stride and one row stride across batches
    if source.stride(-1) != 1 or source.stride(0) != source.shape[1] * source.stride(1):
        return False
    if source.stride(1) % 8 or source.data_ptr() % 16:
        return False
    if not all(t.is_contiguous() for t in [weight, value] + params) or (
        linear_bias is not None and not linear_bias.is_contiguous()
    ):
        return False
    if weight.data_ptr() % 16 or value.data_ptr() % 16 or any(t.data_ptr() % 16 for t in params):
        return False
    if linear_bias is not None and linear_bias.data_ptr() % 8:
        return False
    if not library_available():
        return False
    return is_gfx950(source.device)


def hip_linear_residual_norm(
    source: torch.Tensor,
    weight: torch.Tensor,
    linear_bias: torch.Tensor | None,
    value: torch.Tensor,
    layer_norm: nn.LayerNorm,
    *,
    final_boundary: bool = False,
    block_rows: int,
    num_warps: int,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, str]:
    """``residual = value + round(source @ weight.T + bias)``,
    ``normalized = layer_norm(residual)``, without materializing the update
    (reference: triton_linear_residual_norm, :197-245).  ``final_boundary``
    is accepted for the reference's signature; on a same-dtype stream the
    final boundary's output has the stream dtype too.  ``out`` optionally
    receives the normalized tensor (e.g. a slice of a preallocated output)."""

    del final_boundary
    if not can_use_hip_linear_residual_norm(
        source, weight, linear_bias, value, layer_norm, block_rows=block_rows, num_warps=num_warps
    ):
        raise RuntimeError("HIP Linear residual-norm boundary is ineligible")
    residual = torch.empty_like(value)
    if out is None:
        normalized = torch.empty_like(value)
    elif (
        out.shape == value.shape
        and out.dtype == value.dtype
        and out.device == value.device
        and out.is_contiguous()
        and out.data_ptr() % 16 == 0
    ):
        normalized = out
    else:
        raise RuntimeError("HIP Linear residual-norm output buffer does not match the request")
    width, in_features = weight.shape
    rows = value.shape[0] * value.shape[1]
    try:
        status = load_library().sah_linear_residual_norm(
            source.data_ptr(),
            weight.data_ptr(),
            None if linear_bias is None else linear_bias.data_ptr(),
            value.data_ptr(),
            None if layer_norm.weight is None else layer_norm.weight.data_ptr(),
            None if layer_norm.bias is None else layer_norm.bias.data_ptr(),
            residual.data_ptr(),
            normalized.data_ptr(),
            rows,
            in_features,
            width,
            source.stride(1),
            float(layer_norm.eps),
            dtype_code(value.dtype),
            SAH_NORM_LAYER,
            block_rows,
            num_warps,
            stream_handle(value.device),
        )
        check_status(status, "sah_linear_residual_norm")
    except Exception as exc:
        raise RuntimeError("HIP Linear residual-norm boundary execution failed") from exc
    return residual, normalized, HIP_LINEAR_RESIDUAL_NORM_BACKEND


__all__ = [
    "HIP_LINEAR_RESIDUAL_NORM_BACKEND",
    "NUM_WARPS",
    "SUPPORTED_WIDTHS",
    "block_rows_for",
    "can_use_hip_linear_residual_norm",
    "hip_linear_residual_norm",
    "hip_linear_residual_norm_available",
    "launch_config_is_valid",
    "supported_width",
]
