"""Deployed configuration registry keyed by environment and shape."""

from .environment import EnvironmentFingerprint, ImplementationScope
from .registry import (
    DEFAULT_DEPLOYED_CONFIGS_PATH,
    DEPLOYMENT_SCHEMA_VERSION,
    ShapeFingerprint,
    iter_deployed_configs,
    publish_deployed_config,
    resolve_deployed_config,
)

__all__ = [
    "DEFAULT_DEPLOYED_CONFIGS_PATH",
    "DEPLOYMENT_SCHEMA_VERSION",
    "EnvironmentFingerprint",
    "ImplementationScope",
    "ShapeFingerprint",
    "iter_deployed_configs",
    "publish_deployed_config",
    "resolve_deployed_config",
]
