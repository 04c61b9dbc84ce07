"""CPU restatement of the residual boundary norms (test infrastructure).

residual_layer_norm follows the reference's same-dtype boundary:
``residual_add`` (solution/operators/norm/residual_add.py:28-39: value + update
in the stream dtype) followed by ``nn.LayerNorm`` (biased variance, eps 1e-5;
solution/transformer.py:1629-1632).  The same function covers the mixed
boundary of solution/kernels/norm/triton_mixed_residual.py:41-76 (an fp32
stream with a 16-bit update, promoted exactly; normalized output 16-bit, or
fp32 at the final boundary) through its ``normalized_dtype``.  The statistics
are computed in float64 here, so the oracle is at least as accurate as any
fp32 kernel it checks.
"""

from __future__ import annotations

import numpy as np
import torch


def _stats_layer(x64: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    mean = x64.mean(dim=-1, keepdim=True)
    var = ((x64 - mean) ** 2).mean(dim=-1, keepdim=True)  # biased, like nn.LayerNorm
    return mean, torch.rsqrt(var + eps)


def layer_norm(
    x: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
    eps: float = 1e-5,
    *,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """LayerNorm over the last axis in float64, rounded once to ``out_dtype``."""

    x64 = x.double()
    mean, rstd = _stats_layer(x64, eps)
    y = (x64 - mean) * rstd
    if weight is not None:
        y = y * weight.double()
    if bias is not None:
        y = y + bias.double()
    return y.to(out_dtype or x.dtype)


def rms_norm(
    x: torch.Tensor,
    weight: torch.Tensor | None,
    eps: float = 1e-6,
    *,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * weight`` in float64."""

    x64 = x.double()
    y = x64 * torch.rsqrt((x64 * x64).mean(dim=-1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight.double()
    return y.to(out_dtype or x.dtype)


def residual_layer_norm(
    value: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor | None,
    bias: torch.Tensor | None,
    eps: float = 1e-5,
    *,
    normalized_dtype: torch.dtype | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(residual, normalized) of one boundary.

    The residual is ``value + update`` rounded once to the stream dtype (the
    stream dtype is ``value.dtype``; a 16-bit update is promoted exactly).
    LayerNorm then reads the rounded residual, as the reference does.
    """

    residual = (value.double() + update.double()).to(value.dtype)
    normalized = layer_norm(residual, weight, bias, eps, out_dtype=normalized_dtype or value.dtype)
    return residual, normalized


def residual_rms_norm(
    value: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor | None,
    eps: float = 1e-6,
    *,
    normalized_dtype: torch.dtype | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    residual = (value.double() + update.double()).to(value.dtype)
    return residual, rms_norm(residual, weight, eps, out_dtype=normalized_dtype or value.dtype)


def layer_norm_loop(row: np.ndarray, weight: np.ndarray, bias: np.ndarray, eps: float) -> np.ndarray:
    """Scalar-loop LayerNorm of one row (brute-force pin for tiny widths)."""

    n = len(row)
    mean = 0.0
    for value in row:
        mean += float(value)
    mean /= n
    var = 0.0
    for value in row:
        var += (float(value) - mean) ** 2
    var /= n
    inv = 1.0 / np.sqrt(var + eps)
    return np.array(
        [(float(v) - mean) * inv * float(w) + float(b) for v, w, b in zip(row, weight, bias)]
    )


__all__ = [
    "layer_norm",
    "layer_norm_loop",
    "residual_layer_norm",
    "residual_rms_norm",
    "rms_norm",
]
