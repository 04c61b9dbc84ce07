"""gfx950 fused boundary primitives."""

from .hip_linear_residual_norm import (
    HIP_LINEAR_RESIDUAL_NORM_BACKEND,
    block_rows_for,
    can_use_hip_linear_residual_norm,
    hip_linear_residual_norm,
    hip_linear_residual_norm_available,
    launch_config_is_valid,
    supported_width,
)

__all__ = [
    "HIP_LINEAR_RESIDUAL_NORM_BACKEND",
    "block_rows_for",
    "can_use_hip_linear_residual_norm",
    "hip_linear_residual_norm",
    "hip_linear_residual_norm_available",
    "launch_config_is_valid",
    "supported_width",
]
