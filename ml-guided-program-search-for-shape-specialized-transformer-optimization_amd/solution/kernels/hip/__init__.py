"""ctypes binding of the gfx950 C ABI (include/shape_aware_hip.h)."""

from ._library import (
    ABI_VERSION,
    EXPORTED_SYMBOLS,
    LIBRARY_PATH,
    HipLibraryError,
    is_gfx950,
    library_available,
    load_library,
)

__all__ = [
    "ABI_VERSION",
    "EXPORTED_SYMBOLS",
    "LIBRARY_PATH",
    "HipLibraryError",
    "is_gfx950",
    "library_available",
    "load_library",
]
