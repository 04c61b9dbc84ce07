"""gfx950 projection primitives."""

from .hip_qkv_layout import (
    HIP_QKV_NATIVE_BHSD_BACKEND,
    VALUE_LAYOUTS,
    can_use_hip_qkv_native_bhsd,
    hip_qkv_native_bhsd,
    hip_qkv_native_bhsd_available,
    launch_config_is_valid,
    prevalidated_hip_qkv_native_bhsd,
    supported_shape,
)

__all__ = [
    "HIP_QKV_NATIVE_BHSD_BACKEND",
    "VALUE_LAYOUTS",
    "can_use_hip_qkv_native_bhsd",
    "hip_qkv_native_bhsd",
    "hip_qkv_native_bhsd_available",
    "launch_config_is_valid",
    "prevalidated_hip_qkv_native_bhsd",
    "supported_shape",
]
