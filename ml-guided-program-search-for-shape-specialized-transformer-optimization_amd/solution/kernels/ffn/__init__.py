"""gfx950 FFN primitives."""

from .hip_exact_gelu import (
    HIP_EXACT_GELU_BACKEND,
    can_use_hip_exact_gelu,
    hip_exact_gelu,
    hip_exact_gelu_available,
    prevalidated_hip_exact_gelu,
)
from .hip_linear_gelu import (
    HIP_LINEAR_BACKEND,
    HIP_LINEAR_EXACT_GELU_BACKEND,
    can_use_hip_linear_exact_gelu,
    hip_linear_exact_gelu_available,
    prevalidated_hip_linear,
    prevalidated_hip_linear_exact_gelu,
)

__all__ = [
    "HIP_EXACT_GELU_BACKEND",
    "HIP_LINEAR_BACKEND",
    "HIP_LINEAR_EXACT_GELU_BACKEND",
    "can_use_hip_exact_gelu",
    "can_use_hip_linear_exact_gelu",
    "hip_exact_gelu",
    "hip_exact_gelu_available",
    "hip_linear_exact_gelu_available",
    "prevalidated_hip_exact_gelu",
    "prevalidated_hip_linear",
    "prevalidated_hip_linear_exact_gelu",
]
