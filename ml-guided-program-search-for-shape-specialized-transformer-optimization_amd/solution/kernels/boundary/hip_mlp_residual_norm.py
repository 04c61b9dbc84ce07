"""The whole FFN fused through its residual add and LayerNorm on gfx950.

Counterpart of the reference's fused MLP boundary
(solution/kernels/boundary/triton_ffn_residual_norm.py:1-268): the same
``available / can_use / strict`` functions, the same ``(source,
input_weight, input_bias, output_weight, output_bias, value, layer_norm, *,
final_boundary, block_rows, num_warps)`` call and ``(residual, normalized,
marker)`` return value, the same strictness (ineligible inputs raise
RuntimeError "... ineligible", a failed launch RuntimeError "... execution
failed").  The reference kernel (:44-135) computes GELU(x W1^T + b1) in row
blocks, rounds the hidden block to fp16, multiplies it by W2, rounds the
update to fp16, adds it to the fp32 residual stream and normalizes, without
writing the hidden activation or the update.  This one
(``sah_mlp_residual_norm``, csrc/mlp_norm.hip) does the same on a bf16 or
fp16 stream: the hidden block and the update are rounded to the stream dtype,
and the residual and the normalized rows are the stream dtype (there is no
separate fp32 final-boundary output: the stream is the model dtype).

Domain: width (d_model) 128 or 256 (the reference: 128), ffn_dim a multiple
of 64 (the reference: 128); launch block_rows = 64 rows per workgroup of
num_warps = 4 wavefronts (the reference's residual_norm_launch fields,
solution/transformer.py:849-868).
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

HIP_MLP_RESIDUAL_NORM_BACKEND = "hip_mlp_residual_norm"
SUPPORTED_WIDTHS = frozenset({128, 256})
FFN_MULTIPLE = 64
BLOCK_ROWS = 64
NUM_WARPS = 4
_SUPPORTED_DTYPES = frozenset({torch.bfloat16, torch.float16})


def launch_config_is_valid(width: int, block_rows: int, num_warps: int) -> bool:
    """The launch the gfx950 kernel implements for this width (the C
    library's own table)."""

    values = (width, block_rows, num_warps)
    if any(isinstance(value, bool) or not isinstance(value, int) for value in values):
        return False
    if library_available():
        return bool(load_library().sah_mlp_residual_norm_launch_supported(*values))
    return width in SUPPORTED_WIDTHS and block_rows == BLOCK_ROWS and num_warps == NUM_WARPS


def supported_shape(width: int, ffn_dim: int) -> bool:
    """Model widths with a kernel instantiation."""

    return width in SUPPORTED_WIDTHS and ffn_dim > 0 and ffn_dim % FFN_MULTIPLE == 0


def hip_mlp_residual_norm_available() -> bool:
    """Whether the gfx950 library loads in this process."""

    return library_available()


def can_use_hip_mlp_residual_norm(
    source: torch.Tensor,
    input_weight: torch.Tensor,
    input_bias: torch.Tensor | None,
    output_weight: torch.Tensor,
    output_bias: torch.Tensor | None,
    value: torch.Tensor,
    layer_norm: nn.LayerNorm,
    *,
    block_rows: int = BLOCK_ROWS,
    num_warps: int = NUM_WARPS,
) -> bool:
    """The reference's eligibility rules (triton_ffn_residual_norm.py:140-208)
    with this kernel's dtypes and shapes; never raises."""

    tensors = [source, input_weight, output_weight, value] + [
        t for t in (input_bias, output_bias) if t is not None
    ]
    if not all(isinstance(item, torch.Tensor) for item in tensors):
        return False
    if not isinstance(layer_norm, nn.LayerNorm) or torch.is_grad_enabled():
        return False
    if source.ndim != 3 or value.ndim != 3 or input_weight.ndim != 2 or output_weight.ndim != 2:
        return False
    ffn_dim, width = input_weight.shape
    if not supported_shape(width, ffn_dim) or not launch_config_is_valid(width, block_rows, num_warps):
        return False
    if tuple(output_weight.shape) != (width, ffn_dim):
        return False
    if tuple(source.shape) != tuple(value.shape) or value.shape[-1] != width or source.numel() == 0:
        return False
    if input_bias is not None and tuple(input_bias.shape) != (ffn_dim,):
        return False
    if output_bias is not None and tuple(output_bias.shape) != (width,):
        return False
    if tuple(layer_norm.normalized_shape) != (width,):
        return False
    params = [t for t in (layer_norm.weight, layer_norm.bias) if t is not None]
    if value.dtype not in _SUPPORTED_DTYPES or any(t.dtype != value.dtype for t in tensors + params):
        return False
    if source.device.type != "cuda" or any(t.device != source.device for t in tensors + params):
        return False
    if not all(t.is_contiguous() for t in tensors + params):
        return False
    if any(t.data_ptr() % 16 for t in [source, input_weight, output_weight, value] + params):
        return False
    if any(t is not None and t.data_ptr() % 8 for t in (input_bias, output_bias)):
        return False
    if not library_available():
        return False
    return is_gfx950(source.device)


def hip_mlp_residual_norm(
    source: torch.Tensor,
    input_weight: torch.Tensor,
    input_bias: torch.Tensor | None,
    output_weight: torch.Tensor,
    output_bias: torch.Tensor | None,
    value: torch.Tensor,
    layer_norm: nn.LayerNorm,
    *,
    final_boundary: bool = False,
    block_rows: int = BLOCK_ROWS,
    num_warps: int = NUM_WARPS,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, str]:
    """``residual = value + round(round(GELU(source @ W1.T + b1)) @ W2.T +
    b2)``, ``normalized = layer_norm(residual)``, without materializing the
    hidden activation or the update (reference: triton_ffn_residual_norm,
    :211-268).  ``final_boundary`` is accepted for the reference's signature;
    on a same-dtype stream the final boundary's output has the stream dtype
    too.  ``out`` optionally receives the normalized tensor."""

    if not isinstance(final_boundary, bool):
        raise TypeError("final_boundary must be a bool")
    if not can_use_hip_mlp_residual_norm(
        source,
        input_weight,
        input_bias,
        output_weight,
        output_bias,
        value,
        layer_norm,
        block_rows=block_rows,
        num_warps=num_warps,
    ):
        raise RuntimeError("HIP fused MLP residual-norm boundary is ineligible")
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
        raise RuntimeError("HIP fused MLP residual-norm output buffer does not match the request")
    ffn_dim, width = input_weight.shape
    rows = value.shape[0] * value.shape[1]
    try:
        status = load_library().sah_mlp_residual_norm(
            source.data_ptr(),
            input_weight.data_ptr(),
            None if input_bias is None else input_bias.data_ptr(),
            output_weight.data_ptr(),
            None if output_bias is None else output_bias.data_ptr(),
            value.data_ptr(),
            None if layer_norm.weight is None else layer_norm.weight.data_ptr(),
            None if layer_norm.bias is None else layer_norm.bias.data_ptr(),
            residual.data_ptr(),
            normalized.data_ptr(),
            rows,
            width,
            ffn_dim,
            width,
            float(layer_norm.eps),
            dtype_code(value.dtype),
            SAH_NORM_LAYER,
            block_rows,
            num_warps,
            stream_handle(value.device),
        )
        check_status(status, "sah_mlp_residual_norm")
    except Exception as exc:
        raise RuntimeError("HIP fused MLP residual-norm execution failed") from exc
    return residual, normalized, HIP_MLP_RESIDUAL_NORM_BACKEND


__all__ = [
    "BLOCK_ROWS",
    "FFN_MULTIPLE",
    "HIP_MLP_RESIDUAL_NORM_BACKEND",
    "NUM_WARPS",
    "SUPPORTED_WIDTHS",
    "can_use_hip_mlp_residual_norm",
    "hip_mlp_residual_norm",
    "hip_mlp_residual_norm_available",
    "launch_config_is_valid",
    "supported_shape",
]
