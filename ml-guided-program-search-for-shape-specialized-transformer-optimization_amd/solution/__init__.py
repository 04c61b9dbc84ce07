"""Lazy public solution contract used by the official benchmark.

Mirrors the reference's solution/__init__.py:1-22: only the plugin names
``UserOptimizedTransformer`` and ``copy_model_weights`` are exported, and the
model module is imported on first use.
"""

from __future__ import annotations

from typing import Any

__all__ = ["UserOptimizedTransformer", "copy_model_weights"]


def __getattr__(name: str) -> Any:
    if name not in __all__:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    from .transformer import UserOptimizedTransformer, copy_model_weights

    exports = {
        "UserOptimizedTransformer": UserOptimizedTransformer,
        "copy_model_weights": copy_model_weights,
    }
    globals().update(exports)
    return exports[name]
