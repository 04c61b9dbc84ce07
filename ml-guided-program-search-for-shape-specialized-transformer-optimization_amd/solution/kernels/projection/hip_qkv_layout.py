"""Packed QKV projection straight into head-major Q / K / V on gfx950.

Counterpart of the reference's native-layout QKV projection
(solution/kernels/projection/triton_qkv_layout.py:1-300): the same
``available / can_use / prevalidated / strict`` functions, the same
``(query, key, value, marker)`` return value and the same strictness (an
unsupported launch raises ValueError, ineligible inputs RuntimeError "...
ineligible", a failed launch RuntimeError "... execution failed"; no
fallback).  The reference kernel (:60-115) multiplies x [B*S, D] by the packed
[3D, D] weight in fp32, adds the bias and stores the three D-column blocks as
contiguous [B, H, S, D/H] tensors; this one does the same for bf16 or fp16
operands with one rounding to the operand dtype (``sah_qkv_projection``,
csrc/linear_gelu.hip).

``value_layout="seq_major"`` writes the value block seq-contiguous instead,
into a [B, H, D/H, S8] buffer (S8 = S rounded up to 8) returned as its
[B, H, S, D/H] view with strides (H*dh*S8, dh*S8, 1, S8), for consumers
that want V^T.  The gfx950 attention kernel reads the default [B, H, S, D/H]
V as given (it copies a seq-contiguous V key-major first).

Differences in domain from the reference (fp16, D in {32, 128, 1024},
S in {32, 128, 1024}, H in {1, 2, 4, 16}): bf16 or fp16, any batch and
sequence length with B*S < 2^31, D a multiple of 256, head_dim a multiple of 8.

``*_initial_norm_qkv_native_bhsd`` fuse the model's first LayerNorm into the
projection, the reference's initial-norm / QKV fusion
(solution/kernels/projection/triton_shape07_initial_norm_qkv.py:67-140, fp32
statistics, the normalized row rounded to the operand dtype before the dot,
head-major stores): ``sah_norm_qkv_projection`` forms each row's statistics
exactly as the fused norm kernel does (into an 8-byte-per-token workspace
allocated here from torch's caching allocator), and the projection normalizes
x as it stages it, so the normalized rows never reach HBM and Q / K / V equal,
bit for bit, those of ``sah_norm`` followed by ``sah_qkv_projection``.  Domain: D in
{512, 1024, 2048, 4096} (the reference's kernel serves one shape, B64 S128
D32 H4 fp32, :143-170); the LayerNorm's weight and bias in the operand dtype.
"""

from __future__ import annotations

import torch

from ..hip._library import (
    SAH_QKV_VALUE_BHSD,
    SAH_QKV_VALUE_SEQ_MAJOR,
    check_status,
    dtype_code,
    is_gfx950,
    library_available,
    load_library,
    stream_handle,
)

HIP_QKV_NATIVE_BHSD_BACKEND = "hip_qkv_native_bhsd"
HIP_INITIAL_NORM_QKV_BACKEND = "hip_initial_norm_qkv_native_bhsd"
INITIAL_NORM_WIDTHS = frozenset({512, 1024, 2048, 4096})
DEFAULT_BLOCK_M = 256
DEFAULT_BLOCK_N = 256
DEFAULT_BLOCK_K = 64
DEFAULT_NUM_WARPS = 8
D_MODEL_MULTIPLE = 256
VALUE_LAYOUTS = {"bhsd": SAH_QKV_VALUE_BHSD, "seq_major": SAH_QKV_VALUE_SEQ_MAJOR}
_SUPPORTED_DTYPES = frozenset({torch.bfloat16, torch.float16})


def launch_config_is_valid(block_m: int, block_n: int, block_k: int, num_warps: int) -> bool:
    """The launch the gfx950 kernel implements (the C library's own table)."""

    values = (block_m, block_n, block_k, num_warps)
    if any(isinstance(value, bool) or not isinstance(value, int) for value in values):
        return False
    if library_available():
        return bool(load_library().sah_qkv_launch_supported(*values))
    return values == (DEFAULT_BLOCK_M, DEFAULT_BLOCK_N, DEFAULT_BLOCK_K, DEFAULT_NUM_WARPS)


def _validate_launch_config(block_m: int, block_n: int, block_k: int, num_warps: int) -> None:
    if not launch_config_is_valid(block_m, block_n, block_k, num_warps):
        raise ValueError("unsupported HIP QKV native-layout launch configuration")


def supported_shape(d_model: int, num_heads: int) -> bool:
    """Model widths with a kernel instantiation."""

    return (
        d_model > 0
        and num_heads > 0
        and d_model % D_MODEL_MULTIPLE == 0
        and d_model % num_heads == 0
        and (d_model // num_heads) % 8 == 0
    )


def hip_qkv_native_bhsd_available() -> bool:
    """Whether the gfx950 library loads in this process."""

    return library_available()


def can_use_hip_qkv_native_bhsd(
    hidden_states: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    num_heads: int,
    block_m: int = DEFAULT_BLOCK_M,
    block_n: int = DEFAULT_BLOCK_N,
    block_k: int = DEFAULT_BLOCK_K,
    num_warps: int = DEFAULT_NUM_WARPS,
) -> bool:
    """The reference's eligibility rules (triton_qkv_layout.py:127-167) with
    this kernel's dtypes and shapes; never raises."""

    if not launch_config_is_valid(block_m, block_n, block_k, num_warps):
        return False
    tensors = [hidden_states, weight] + ([] if bias is None else [bias])
    if not all(isinstance(item, torch.Tensor) for item in tensors):
        return False
    if isinstance(num_heads, bool) or not isinstance(num_heads, int):
        return False
    # No autograd: refused while grad is enabled.  Under no_grad /
    # inference_mode the model's parameters (requires_grad=True) are plain
    # operands; the reference passes detached fp16 shadows instead.
    if torch.is_grad_enabled():
        return False
    if hidden_states.device.type != "cuda" or any(t.device != hidden_states.device for t in tensors):
        return False
    if hidden_states.ndim != 3 or hidden_states.dtype not in _SUPPORTED_DTYPES:
        return False
    batch, seq_len, d_model = hidden_states.shape
    if batch <= 0 or seq_len <= 0 or batch * seq_len >= 2**31:
        return False
    if not supported_shape(d_model, num_heads):
        return False
    if weight.shape != (3 * d_model, d_model) or (bias is not None and bias.shape != (3 * d_model,)):
        return False
    if any(t.dtype != hidden_states.dtype for t in tensors):
        return False
    if not all(t.is_contiguous() for t in tensors):
        return False
    if hidden_states.data_ptr() % 16 or weight.data_ptr() % 16 or (bias is not None and bias.data_ptr() % 8):
        return False
    if not library_available():
        return False
    return is_gfx950(hidden_states.device)


def _layer_norm_parameters(layer_norm: torch.nn.LayerNorm) -> tuple[torch.Tensor, torch.Tensor, float] | None:
    weight, bias = layer_norm.weight, layer_norm.bias
    if not isinstance(weight, torch.Tensor) or not isinstance(bias, torch.Tensor):
        return None
    return weight, bias, float(layer_norm.eps)


def can_use_hip_initial_norm_qkv_native_bhsd(
    hidden_states: torch.Tensor,
    layer_norm: torch.nn.LayerNorm,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    num_heads: int,
    block_m: int = DEFAULT_BLOCK_M,
    block_n: int = DEFAULT_BLOCK_N,
    block_k: int = DEFAULT_BLOCK_K,
    num_warps: int = DEFAULT_NUM_WARPS,
) -> bool:
    """The projection's rules plus the LayerNorm's: an affine LayerNorm over
    the last dimension of a width the statistics are instantiated for, its
    weight and bias contiguous and in the operand dtype, a finite eps >= 0.
    Never raises."""

    if not isinstance(layer_norm, torch.nn.LayerNorm):
        return False
    parameters = _layer_norm_parameters(layer_norm)
    if parameters is None:
        return False
    norm_weight, norm_bias, eps = parameters
    if not isinstance(hidden_states, torch.Tensor) or hidden_states.ndim != 3:
        return False
    d_model = hidden_states.shape[-1]
    if tuple(layer_norm.normalized_shape) != (d_model,) or d_model not in INITIAL_NORM_WIDTHS:
        return False
    if not (eps >= 0.0 and eps < float("inf")):
        return False
    for tensor in (norm_weight, norm_bias):
        if tensor.shape != (d_model,) or tensor.dtype != hidden_states.dtype:
            return False
        if tensor.device != hidden_states.device or not tensor.is_contiguous() or tensor.data_ptr() % 16:
            return False
    return can_use_hip_qkv_native_bhsd(
        hidden_states,
        weight,
        bias,
        num_heads=num_heads,
        block_m=block_m,
        block_n=block_n,
        block_k=block_k,
        num_warps=num_warps,
    )


def prevalidated_hip_qkv_native_bhsd(
    hidden_states: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    num_heads: int,
    block_m: int = DEFAULT_BLOCK_M,
    block_n: int = DEFAULT_BLOCK_N,
    block_k: int = DEFAULT_BLOCK_K,
    num_warps: int = DEFAULT_NUM_WARPS,
    value_layout: str = "bhsd",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, str]:
    """Project after the caller established eligibility (reference:
    prevalidated_triton_qkv_native_bhsd, :170-230).  Returns (query, key,
    value, marker) as [B, H, S, D/H] tensors; query and key contiguous, value
    contiguous or the seq-contiguous view described in the module docstring."""

    _validate_launch_config(block_m, block_n, block_k, num_warps)
    if value_layout not in VALUE_LAYOUTS:
        raise ValueError(f"unknown value layout {value_layout!r}; expected one of {sorted(VALUE_LAYOUTS)}")
    # The kernel reads x as [B*S, D] rows and the packed weight as [3D, D]:
    # anything else would be read wrongly, so it is refused, not computed.
    if not can_use_hip_qkv_native_bhsd(
        hidden_states,
        weight,
        bias,
        num_heads=num_heads,
        block_m=block_m,
        block_n=block_n,
        block_k=block_k,
        num_warps=num_warps,
    ):
        raise RuntimeError("HIP QKV native-layout projection inputs are ineligible for the gfx950 kernel")
    return _launch(
        hidden_states, None, weight, bias, num_heads, (block_m, block_n, block_k, num_warps), value_layout
    ) + (HIP_QKV_NATIVE_BHSD_BACKEND,)


def prevalidated_hip_initial_norm_qkv_native_bhsd(
    hidden_states: torch.Tensor,
    layer_norm: torch.nn.LayerNorm,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    num_heads: int,
    block_m: int = DEFAULT_BLOCK_M,
    block_n: int = DEFAULT_BLOCK_N,
    block_k: int = DEFAULT_BLOCK_K,
    num_warps: int = DEFAULT_NUM_WARPS,
    value_layout: str = "bhsd",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, str]:
    """``layer_norm(hidden_states)`` projected into head-major Q / K / V in
    one kernel; the normalized rows never reach HBM (reference: the fused
    initial-norm QKV launch, triton_shape07_initial_norm_qkv.py:173-218).
    Same return value and errors as :func:`prevalidated_hip_qkv_native_bhsd`."""

    _validate_launch_config(block_m, block_n, block_k, num_warps)
    if value_layout not in VALUE_LAYOUTS:
        raise ValueError(f"unknown value layout {value_layout!r}; expected one of {sorted(VALUE_LAYOUTS)}")
    if not can_use_hip_initial_norm_qkv_native_bhsd(
        hidden_states,
        layer_norm,
        weight,
        bias,
        num_heads=num_heads,
        block_m=block_m,
        block_n=block_n,
        block_k=block_k,
        num_warps=num_warps,
    ):
        raise RuntimeError("HIP initial-norm QKV projection inputs are ineligible for the gfx950 kernel")
    return _launch(
        hidden_states,
        _layer_norm_parameters(layer_norm),
        weight,
        bias,
        num_heads,
        (block_m, block_n, block_k, num_warps),
        value_layout,
    ) + (HIP_INITIAL_NORM_QKV_BACKEND,)


def _launch(
    hidden_states: torch.Tensor,
    layer_norm: tuple[torch.Tensor, torch.Tensor, float] | None,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    num_heads: int,
    launch: tuple[int, int, int, int],
    value_layout: str,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    batch, seq_len, d_model = hidden_states.shape
    head_dim = d_model // num_heads
    shape = (batch, num_heads, seq_len, head_dim)
    device, dtype = hidden_states.device, hidden_states.dtype
    query = torch.empty(shape, device=device, dtype=dtype)
    key = torch.empty_like(query)
    if value_layout == "seq_major":
        seq_stride = (seq_len + 7) // 8 * 8
        storage = torch.empty((batch, num_heads, head_dim, seq_stride), device=device, dtype=dtype)
        value = storage[..., :seq_len].transpose(-1, -2)
    else:
        seq_stride = 0
        value = torch.empty_like(query)
    operands = (
        weight.data_ptr(),
        None if bias is None else bias.data_ptr(),
        query.data_ptr(),
        key.data_ptr(),
        value.data_ptr(),
        batch,
        seq_len,
        d_model,
        num_heads,
        hidden_states.stride(1),
        VALUE_LAYOUTS[value_layout],
        seq_stride,
        dtype_code(dtype),
        *launch,
        stream_handle(device),
    )
    library = load_library()
    try:
        if layer_norm is None:
            status = library.sah_qkv_projection(hidden_states.data_ptr(), *operands)
            check_status(status, "sah_qkv_projection")
        else:
            norm_weight, norm_bias, eps = layer_norm
            workspace_bytes = int(library.sah_norm_qkv_workspace_bytes(batch, seq_len))
            workspace = torch.empty(max(workspace_bytes, 16), device=device, dtype=torch.uint8)
            status = library.sah_norm_qkv_projection(
                hidden_states.data_ptr(),
                norm_weight.data_ptr(),
                norm_bias.data_ptr(),
                eps,
                *operands[:-1],
                workspace.data_ptr(),
                workspace.numel(),
                operands[-1],
            )
            check_status(status, "sah_norm_qkv_projection")
    except Exception as exc:
        raise RuntimeError("HIP QKV native-layout projection execution failed") from exc
    return query, key, value


def hip_qkv_native_bhsd(
    hidden_states: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    num_heads: int,
    block_m: int = DEFAULT_BLOCK_M,
    block_n: int = DEFAULT_BLOCK_N,
    block_k: int = DEFAULT_BLOCK_K,
    num_warps: int = DEFAULT_NUM_WARPS,
    value_layout: str = "bhsd",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, str]:
    """Strict entry (reference: triton_qkv_native_bhsd, :233-265): checks
    eligibility first and raises RuntimeError "... ineligible" otherwise."""

    _validate_launch_config(block_m, block_n, block_k, num_warps)
    if not can_use_hip_qkv_native_bhsd(
        hidden_states,
        weight,
        bias,
        num_heads=num_heads,
        block_m=block_m,
        block_n=block_n,
        block_k=block_k,
        num_warps=num_warps,
    ):
        raise RuntimeError("HIP QKV native-layout projection is ineligible")
    return prevalidated_hip_qkv_native_bhsd(
        hidden_states,
        weight,
        bias,
        num_heads=num_heads,
        block_m=block_m,
        block_n=block_n,
        block_k=block_k,
        num_warps=num_warps,
        value_layout=value_layout,
    )


__all__ = [
    "DEFAULT_BLOCK_K",
    "DEFAULT_BLOCK_M",
    "DEFAULT_BLOCK_N",
    "DEFAULT_NUM_WARPS",
    "HIP_INITIAL_NORM_QKV_BACKEND",
    "HIP_QKV_NATIVE_BHSD_BACKEND",
    "INITIAL_NORM_WIDTHS",
    "VALUE_LAYOUTS",
    "can_use_hip_initial_norm_qkv_native_bhsd",
    "can_use_hip_qkv_native_bhsd",
    "hip_qkv_native_bhsd",
    "hip_qkv_native_bhsd_available",
    "launch_config_is_valid",
    "prevalidated_hip_initial_norm_qkv_native_bhsd",
    "prevalidated_hip_qkv_native_bhsd",
    "supported_shape",
]
