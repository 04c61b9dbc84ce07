"""Fused residual + LayerNorm/RMSNorm on gfx950 through the C ABI.

Counterparts of the reference's norm primitives with the same call shapes,
return values (``(residual, normalized, marker)``) and strictness (no silent
fallback; ineligible inputs raise RuntimeError, bad launch values ValueError):

* :func:`hip_residual_layer_norm` - the residual boundary.  With a same-dtype
  stream it computes what the reference's TORCH boundary computes
  (residual_add + nn.LayerNorm, solution/operators/norm/residual_add.py:28-39,
  solution/transformer.py:1629-1632) and what its fp32 Triton kernel computes
  (solution/kernels/norm/triton_residual.py:110-148); with an fp32 stream and
  a 16-bit update it is the mixed boundary
  (solution/kernels/norm/triton_mixed_residual.py:114-157), whose normalized
  output is 16-bit except at the final boundary.
* :func:`hip_layer_norm` - the layer-0 initial norm
  (solution/kernels/norm/triton_initial.py:101-135).
* :func:`hip_residual_rms_norm` / :func:`hip_rms_norm` - the same kernel with
  RMS statistics, ``y = x * rsqrt(mean(x^2) + eps) * weight``.
"""

from __future__ import annotations

import torch
from torch import nn

from ..hip._library import (
    SAH_NORM_LAYER,
    SAH_NORM_RMS,
    HipLibraryError,
    check_status,
    dtype_code,
    is_gfx950,
    library_available,
    load_library,
    stream_handle,
)

HIP_RESIDUAL_LAYER_NORM_BACKEND = "hip_residual_layer_norm"
HIP_RESIDUAL_RMS_NORM_BACKEND = "hip_residual_rms_norm"
HIP_LAYER_NORM_BACKEND = "hip_layer_norm"
HIP_RMS_NORM_BACKEND = "hip_rms_norm"

DEFAULT_BLOCK_ROWS = 4
DEFAULT_NUM_WARPS = 4
SUPPORTED_NUM_WARPS = frozenset({1, 2, 4, 8})
_MAX_BLOCK_ROWS = 64

_HALF = (torch.float16, torch.bfloat16)
# (value/residual dtype, update dtype, normalized dtype) implemented by the kernel.
RESIDUAL_DTYPE_COMBINATIONS = frozenset(
    {
        (torch.bfloat16, torch.bfloat16, torch.bfloat16),
        (torch.float16, torch.float16, torch.float16),
        (torch.float32, torch.float32, torch.float32),
        (torch.float32, torch.float16, torch.float16),
        (torch.float32, torch.float16, torch.float32),
        (torch.float32, torch.bfloat16, torch.bfloat16),
        (torch.float32, torch.bfloat16, torch.float32),
    }
)
# (value dtype, normalized dtype) for the norm without residual.
NORM_DTYPE_COMBINATIONS = frozenset(
    {
        (torch.bfloat16, torch.bfloat16),
        (torch.float16, torch.float16),
        (torch.float32, torch.float32),
        (torch.float32, torch.float16),
        (torch.float32, torch.bfloat16),
    }
)


def launch_config_is_valid(block_rows: int, num_warps: int) -> bool:
    """Rows per workgroup and wavefronts per workgroup the kernel accepts."""

    values = (block_rows, num_warps)
    return bool(
        not any(isinstance(value, bool) for value in values)
        and all(isinstance(value, int) for value in values)
        and num_warps in SUPPORTED_NUM_WARPS
        and 0 < block_rows <= _MAX_BLOCK_ROWS
        and block_rows % num_warps == 0
    )


def _validate_launch_config(block_rows: int, num_warps: int) -> None:
    if not launch_config_is_valid(block_rows, num_warps):
        raise ValueError("unsupported HIP residual norm launch configuration")


def supported_width(width: int, value_dtype: torch.dtype) -> bool:
    """Widths with a kernel instantiation: 64 lanes x 16 bytes x {1, 2, 4, 8,
    16}, and the rows narrower than one such pass (width 128; width 256 for
    16-bit values), read with 4- or 8-byte accesses."""

    element_size = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}.get(value_dtype)
    if element_size is None:
        return False
    per_iteration = 64 * (16 // element_size)
    if width in (128, 256) and width < per_iteration:
        return True
    if width <= 0 or width % per_iteration:
        return False
    return width // per_iteration in {1, 2, 4, 8, 16}


def hip_residual_norm_available() -> bool:
    """Whether the gfx950 library loads in this process."""

    return library_available()


def _param_dtype(
    weight: torch.Tensor | None, bias: torch.Tensor | None, value_dtype: torch.dtype
) -> torch.dtype | None:
    dtypes = {t.dtype for t in (weight, bias) if t is not None}
    if not dtypes:
        return torch.float32
    if len(dtypes) != 1:
        return None
    (dtype,) = dtypes
    if dtype == torch.float32 or dtype == value_dtype:
        return dtype
    return None


def _params_ok(
    value: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
) -> bool:
    width = value.shape[-1]
    for parameter in (weight, bias):
        if parameter is None:
            continue
        if parameter.shape != (width,) or parameter.device != value.device:
            return False
        if not parameter.is_contiguous() or parameter.data_ptr() % 16:
            return False
        if parameter.requires_grad and torch.is_grad_enabled():
            return False
    return _param_dtype(weight, bias, value.dtype) is not None


def _device_ok(*tensors: torch.Tensor) -> bool:
    device = tensors[0].device
    if device.type != "cuda":
        return False
    return all(t.device == device for t in tensors) and is_gfx950(device)


def can_use_hip_residual_norm(
    value: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
    *,
    normalized_dtype: torch.dtype | None = None,
) -> bool:
    """Whether the fused residual kernel implements this request."""

    normalized_dtype = value.dtype if normalized_dtype is None else normalized_dtype
    if (value.dtype, update.dtype, normalized_dtype) not in RESIDUAL_DTYPE_COMBINATIONS:
        return False
    if value.shape != update.shape or value.ndim < 1:
        return False
    if not supported_width(value.shape[-1], value.dtype):
        return False
    if not value.is_contiguous() or not update.is_contiguous():
        return False
    if value.data_ptr() % 16 or update.data_ptr() % 16:
        return False
    if torch.is_grad_enabled() and (value.requires_grad or update.requires_grad):
        return False
    if not _params_ok(value, weight, bias):
        return False
    if not library_available():
        return False
    return _device_ok(value, update)


def can_use_hip_norm(
    value: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
    *,
    normalized_dtype: torch.dtype | None = None,
) -> bool:
    """Whether the no-residual norm kernel implements this request."""

    normalized_dtype = value.dtype if normalized_dtype is None else normalized_dtype
    if (value.dtype, normalized_dtype) not in NORM_DTYPE_COMBINATIONS:
        return False
    if value.ndim < 1 or not supported_width(value.shape[-1], value.dtype):
        return False
    if not value.is_contiguous() or value.data_ptr() % 16:
        return False
    if torch.is_grad_enabled() and value.requires_grad:
        return False
    if not _params_ok(value, weight, bias):
        return False
    if not library_available():
        return False
    return _device_ok(value)


def _check_out(
    out: torch.Tensor | None, like: torch.Tensor, dtype: torch.dtype
) -> torch.Tensor:
    if out is None:
        return torch.empty(like.shape, dtype=dtype, device=like.device)
    if (
        out.shape != like.shape
        or out.dtype != dtype
        or out.device != like.device
        or not out.is_contiguous()
        or out.data_ptr() % 16
    ):
        raise RuntimeError("HIP norm output buffer does not match the request")
    return out


def _launch_residual(
    value: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
    eps: float,
    normalized_dtype: torch.dtype,
    norm_kind: int,
    block_rows: int,
    num_warps: int,
    out: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor]:
    library = load_library()
    width = value.shape[-1]
    rows = value.numel() // width
    residual = torch.empty_like(value)
    normalized = _check_out(out, value, normalized_dtype)
    param_dtype = _param_dtype(weight, bias, value.dtype)
    assert param_dtype is not None
    status = library.sah_residual_norm(
        value.data_ptr(),
        update.data_ptr(),
        None if weight is None else weight.data_ptr(),
        None if bias is None else bias.data_ptr(),
        residual.data_ptr(),
        normalized.data_ptr(),
        rows,
        width,
        float(eps),
        dtype_code(value.dtype),
        dtype_code(update.dtype),
        dtype_code(normalized_dtype),
        dtype_code(param_dtype),
        norm_kind,
        block_rows,
        num_warps,
        stream_handle(value.device),
    )
    check_status(status, "sah_residual_norm")
    return residual, normalized


def _launch_norm(
    value: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
    eps: float,
    normalized_dtype: torch.dtype,
    norm_kind: int,
    block_rows: int,
    num_warps: int,
    out: torch.Tensor | None,
) -> torch.Tensor:
    library = load_library()
    width = value.shape[-1]
    rows = value.numel() // width
    normalized = _check_out(out, value, normalized_dtype)
    param_dtype = _param_dtype(weight, bias, value.dtype)
    assert param_dtype is not None
    status = library.sah_norm(
        value.data_ptr(),
        None if weight is None else weight.data_ptr(),
        None if bias is None else bias.data_ptr(),
        normalized.data_ptr(),
        rows,
        width,
        float(eps),
        dtype_code(value.dtype),
        dtype_code(normalized_dtype),
        dtype_code(param_dtype),
        norm_kind,
        block_rows,
        num_warps,
        stream_handle(value.device),
    )
    check_status(status, "sah_norm")
    return normalized


def _layer_norm_params(
    layer_norm: nn.LayerNorm, width: int
) -> tuple[torch.Tensor | None, torch.Tensor | None, float]:
    if not isinstance(layer_norm, nn.LayerNorm):
        raise RuntimeError("HIP norm requires an nn.LayerNorm module")
    if tuple(layer_norm.normalized_shape) != (width,):
        raise RuntimeError("HIP norm requires a LayerNorm over the last axis")
    return layer_norm.weight, layer_norm.bias, float(layer_norm.eps)


def hip_residual_layer_norm(
    value: torch.Tensor,
    update: torch.Tensor,
    layer_norm: nn.LayerNorm,
    *,
    normalized_dtype: torch.dtype | None = None,
    block_rows: int = DEFAULT_BLOCK_ROWS,
    num_warps: int = DEFAULT_NUM_WARPS,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, str]:
    """``residual = value + update``; ``normalized = layer_norm(residual)``.

    ``normalized_dtype`` defaults to the stream dtype; an fp32 stream with a
    16-bit update selects the mixed boundary (pass the 16-bit dtype for an
    intermediate boundary and float32 for the final one).  ``out`` optionally
    receives the normalized tensor (e.g. a slice of a preallocated output).
    """

    _validate_launch_config(block_rows, num_warps)
    weight, bias, eps = _layer_norm_params(layer_norm, value.shape[-1])
    normalized_dtype = value.dtype if normalized_dtype is None else normalized_dtype
    if not can_use_hip_residual_norm(
        value, update, weight, bias, normalized_dtype=normalized_dtype
    ):
        raise RuntimeError("HIP residual LayerNorm is ineligible for the requested inputs")
    try:
        residual, normalized = _launch_residual(
            value, update, weight, bias, eps, normalized_dtype, SAH_NORM_LAYER,
            block_rows, num_warps, out,
        )
    except HipLibraryError as exc:
        raise RuntimeError("HIP residual LayerNorm execution failed") from exc
    return residual, normalized, HIP_RESIDUAL_LAYER_NORM_BACKEND


def hip_residual_rms_norm(
    value: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor | None,
    *,
    eps: float = 1e-6,
    normalized_dtype: torch.dtype | None = None,
    block_rows: int = DEFAULT_BLOCK_ROWS,
    num_warps: int = DEFAULT_NUM_WARPS,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, str]:
    """``residual = value + update``; ``normalized = rms_norm(residual) * weight``."""

    _validate_launch_config(block_rows, num_warps)
    normalized_dtype = value.dtype if normalized_dtype is None else normalized_dtype
    if not can_use_hip_residual_norm(
        value, update, weight, None, normalized_dtype=normalized_dtype
    ):
        raise RuntimeError("HIP residual RMSNorm is ineligible for the requested inputs")
    try:
        residual, normalized = _launch_residual(
            value, update, weight, None, eps, normalized_dtype, SAH_NORM_RMS,
            block_rows, num_warps, out,
        )
    except HipLibraryError as exc:
        raise RuntimeError("HIP residual RMSNorm execution failed") from exc
    return residual, normalized, HIP_RESIDUAL_RMS_NORM_BACKEND


def hip_layer_norm(
    value: torch.Tensor,
    layer_norm: nn.LayerNorm,
    *,
    normalized_dtype: torch.dtype | None = None,
    block_rows: int = DEFAULT_BLOCK_ROWS,
    num_warps: int = DEFAULT_NUM_WARPS,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, str]:
    """``normalized = layer_norm(value)`` (the layer-0 initial norm)."""

    _validate_launch_config(block_rows, num_warps)
    weight, bias, eps = _layer_norm_params(layer_norm, value.shape[-1])
    normalized_dtype = value.dtype if normalized_dtype is None else normalized_dtype
    if not can_use_hip_norm(value, weight, bias, normalized_dtype=normalized_dtype):
        raise RuntimeError("HIP LayerNorm is ineligible for the requested input")
    try:
        normalized = _launch_norm(
            value, weight, bias, eps, normalized_dtype, SAH_NORM_LAYER,
            block_rows, num_warps, out,
        )
    except HipLibraryError as exc:
        raise RuntimeError("HIP LayerNorm execution failed") from exc
    return normalized, HIP_LAYER_NORM_BACKEND


def hip_rms_norm(
    value: torch.Tensor,
    weight: torch.Tensor | None,
    *,
    eps: float = 1e-6,
    normalized_dtype: torch.dtype | None = None,
    block_rows: int = DEFAULT_BLOCK_ROWS,
    num_warps: int = DEFAULT_NUM_WARPS,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, str]:
    """``normalized = value * rsqrt(mean(value^2) + eps) * weight``."""

    _validate_launch_config(block_rows, num_warps)
    normalized_dtype = value.dtype if normalized_dtype is None else normalized_dtype
    if not can_use_hip_norm(value, weight, None, normalized_dtype=normalized_dtype):
        raise RuntimeError("HIP RMSNorm is ineligible for the requested input")
    try:
        normalized = _launch_norm(
            value, weight, None, eps, normalized_dtype, SAH_NORM_RMS,
            block_rows, num_warps, out,
        )
    except HipLibraryError as exc:
        raise RuntimeError("HIP RMSNorm execution failed") from exc
    return normalized, HIP_RMS_NORM_BACKEND


__all__ = [
    "DEFAULT_BLOCK_ROWS",
    "DEFAULT_NUM_WARPS",
    "HIP_LAYER_NORM_BACKEND",
    "HIP_RESIDUAL_LAYER_NORM_BACKEND",
    "HIP_RESIDUAL_RMS_NORM_BACKEND",
    "HIP_RMS_NORM_BACKEND",
    "NORM_DTYPE_COMBINATIONS",
    "RESIDUAL_DTYPE_COMBINATIONS",
    "can_use_hip_norm",
    "can_use_hip_residual_norm",
    "hip_layer_norm",
    "hip_residual_layer_norm",
    "hip_residual_norm_available",
    "hip_residual_rms_norm",
    "hip_rms_norm",
    "launch_config_is_valid",
    "supported_width",
]
