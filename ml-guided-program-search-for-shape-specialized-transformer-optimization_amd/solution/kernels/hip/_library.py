"""ctypes binding of the gfx950 C ABI declared in include/shape_aware_hip.h.

The shared library is built in-tree (``csrc/build.py``) and linked against the
HIP runtime inside the installed PyTorch, so the raw ``hipStream_t`` handles
of torch streams and the device pointers of torch tensors are passed straight
through.  Nothing here falls back to another implementation: a missing or
stale library raises :class:`HipLibraryError`.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

PACKAGE_ROOT = Path(__file__).resolve().parents[3]
LIBRARY_PATH = PACKAGE_ROOT / "lib" / "libshape_aware_hip.so"
ABI_VERSION = 1

SAH_OK = 0
SAH_ERR_INVALID_ARGUMENT = 1
SAH_ERR_UNSUPPORTED = 2
SAH_ERR_HIP = 3
SAH_ERR_WORKSPACE = 4

SAH_ACTIVATION_NONE = 0
SAH_ACTIVATION_GELU_EXACT = 1
SAH_QKV_VALUE_BHSD = 0
SAH_QKV_VALUE_SEQ_MAJOR = 1
SAH_NORM_LAYER = 0
SAH_NORM_RMS = 1

_DTYPE_CODES = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
}

# Every exported entry point with its ctypes signature (argtypes, restype).
_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_SIGNATURES: dict[str, tuple[list[object], object]] = {
    "sah_abi_version": ([], _int),
    "sah_last_error": ([], ctypes.c_char_p),
    "sah_causal_attention_bsd": (
        [_ptr, _ptr, _ptr, _ptr]
        + [_i64] * 4
        + [_i64] * 3
        + [_i64] * 3
        + [_i64] * 4
        + [_i64] * 2
        + [ctypes.c_float, _int]
        + [_int] * 4
        + [_ptr, ctypes.c_size_t, _ptr],
        _int,
    ),
    "sah_causal_attention_bsd_static_workspace": (
        [_ptr, _ptr, _ptr, _ptr]
        + [_i64] * 4
        + [_i64] * 3
        + [_i64] * 3
        + [_i64] * 4
        + [_i64] * 2
        + [ctypes.c_float, _int]
        + [_int] * 4
        + [_ptr],
        _int,
    ),
    "sah_causal_attention_workspace_bytes": ([_i64] * 6 + [_int], ctypes.c_size_t),
    "sah_causal_attention_launch_supported": ([_int] * 4, _int),
    "sah_residual_norm": (
        [_ptr] * 6 + [_i64, _i64, ctypes.c_float] + [_int] * 7 + [_ptr],
        _int,
    ),
    "sah_norm": (
        [_ptr] * 4 + [_i64, _i64, ctypes.c_float] + [_int] * 6 + [_ptr],
        _int,
    ),
    "sah_linear": ([_ptr] * 4 + [_i64] * 5 + [_int] * 2 + [_int] * 5 + [_ptr], _int),
    "sah_linear_launch_supported": ([_int] * 5, _int),
    "sah_gelu": ([_ptr, _ptr, _i64, _int, _int, _int, _ptr], _int),
    "sah_gelu_launch_supported": ([_int] * 2, _int),
    "sah_qkv_projection": (
        [_ptr] * 6 + [_i64] * 5 + [_int, _i64] + [_int] * 5 + [_ptr],
        _int,
    ),
    "sah_norm_qkv_projection": (
        [_ptr] * 3 + [ctypes.c_float] + [_ptr] * 5 + [_i64] * 5 + [_int, _i64] + [_int] * 5
        + [_ptr, ctypes.c_size_t, _ptr],
        _int,
    ),
    "sah_norm_qkv_workspace_bytes": ([_i64, _i64], ctypes.c_size_t),
    "sah_qkv_launch_supported": ([_int] * 4, _int),
    "sah_linear_residual_norm": (
        [_ptr] * 8 + [_i64] * 4 + [ctypes.c_float] + [_int] * 4 + [_ptr],
        _int,
    ),
    "sah_linear_residual_norm_launch_supported": ([_i64, _int, _int], _int),
    "sah_mlp_residual_norm": (
        [_ptr] * 10 + [_i64] * 4 + [ctypes.c_float] + [_int] * 4 + [_ptr],
        _int,
    ),
    "sah_mlp_residual_norm_launch_supported": ([_i64, _int, _int], _int),
}
EXPORTED_SYMBOLS = tuple(_SIGNATURES)
# SAH_ATTENTION_STATIC_WORKSPACE_BYTES of the header: the device array behind
# sah_causal_attention_bsd_static_workspace.
ATTENTION_STATIC_WORKSPACE_BYTES = 64 << 20


class HipLibraryError(RuntimeError):
    """The gfx950 library is missing, stale or returned an error status."""


_lock = threading.Lock()
_library: ctypes.CDLL | None = None
_load_error: str | None = None


def _load() -> ctypes.CDLL:
    if not LIBRARY_PATH.exists():
        raise HipLibraryError(
            f"{LIBRARY_PATH} is not built; run csrc/build.py (or __graft_entry__.build())"
        )
    library = ctypes.CDLL(str(LIBRARY_PATH), mode=ctypes.RTLD_LOCAL)
    for name, (argtypes, restype) in _SIGNATURES.items():
        function = getattr(library, name)
        function.argtypes = argtypes
        function.restype = restype
    version = library.sah_abi_version()
    if version != ABI_VERSION:
        raise HipLibraryError(
            f"{LIBRARY_PATH} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
        )
    return library


def load_library() -> ctypes.CDLL:
    """Return the loaded library or raise :class:`HipLibraryError`."""

    global _library, _load_error
    if _library is not None:
        return _library
    with _lock:
        if _library is None:
            try:
                _library = _load()
                _load_error = None
            except (OSError, AttributeError, HipLibraryError) as exc:
                _load_error = str(exc)
                raise HipLibraryError(str(exc)) from exc
    return _library


def library_available() -> bool:
    """Whether the library loads in this process (never raises)."""

    try:
        load_library()
    except HipLibraryError:
        return False
    return True


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"dtype {dtype} has no gfx950 kernel") from None


def check_status(status: int, what: str) -> None:
    """Raise with the library's message for a nonzero status."""

    if status == SAH_OK:
        return
    message = load_library().sah_last_error().decode("utf-8", "replace")
    raise HipLibraryError(f"{what} failed with status {status}: {message}")


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def stream_handle(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``.  Read as the
    raw handle, without building a torch Stream object: every kernel launch
    asks for it, and on the C2 forward (~60 launches in 0.9 ms) the host's
    per-launch time is as long as the GPU's."""

    return int(torch._C._cuda_getCurrentRawStream(_device_index(device)))


# gfx950 or not, per device index: device properties do not change within a
# process, and every operator's eligibility check asks.
_GFX950_BY_INDEX: dict[int, bool] = {}


def is_gfx950(device: torch.device) -> bool:
    """Whether ``device`` is a CDNA4 (gfx950) GPU visible to torch."""

    if device.type != "cuda" or torch.version.hip is None:
        return False
    if not _GFX950_BY_INDEX and not torch.cuda.is_available():
        return False
    index = _device_index(device)
    known = _GFX950_BY_INDEX.get(index)
    if known is None:
        arch = getattr(torch.cuda.get_device_properties(index), "gcnArchName", "")
        known = str(arch).split(":")[0] == "gfx950"
        _GFX950_BY_INDEX[index] = known
    return known


__all__ = [
    "ABI_VERSION",
    "EXPORTED_SYMBOLS",
    "HipLibraryError",
    "LIBRARY_PATH",
    "SAH_ACTIVATION_GELU_EXACT",
    "SAH_ACTIVATION_NONE",
    "SAH_QKV_VALUE_BHSD",
    "SAH_QKV_VALUE_SEQ_MAJOR",
    "SAH_NORM_LAYER",
    "SAH_NORM_RMS",
    "check_status",
    "dtype_code",
    "is_gfx950",
    "library_available",
    "load_library",
    "stream_handle",
]
