"""gfx950 residual-plus-norm primitives."""

from .hip_residual import (
    HIP_LAYER_NORM_BACKEND,
    HIP_RESIDUAL_LAYER_NORM_BACKEND,
    HIP_RESIDUAL_RMS_NORM_BACKEND,
    HIP_RMS_NORM_BACKEND,
    can_use_hip_norm,
    can_use_hip_residual_norm,
    hip_layer_norm,
    hip_residual_layer_norm,
    hip_residual_norm_available,
    hip_residual_rms_norm,
    hip_rms_norm,
)

__all__ = [
    "HIP_LAYER_NORM_BACKEND",
    "HIP_RESIDUAL_LAYER_NORM_BACKEND",
    "HIP_RESIDUAL_RMS_NORM_BACKEND",
    "HIP_RMS_NORM_BACKEND",
    "can_use_hip_norm",
    "can_use_hip_residual_norm",
    "hip_layer_norm",
    "hip_residual_layer_norm",
    "hip_residual_norm_available",
    "hip_residual_rms_norm",
    "hip_rms_norm",
]
