"""Forward-only causal attention (head_dim 64) on gfx950 through the C ABI.

Drop-in counterpart of the reference's Triton streaming kernel module
(solution/shape14/triton_streaming_dh64.py:1-398): the same public function
shapes (``*_available``, ``can_use_*``, ``prevalidated_*_bsd`` returning
``(output, marker)``, strict ``*_bsd``), the same argument meaning and the same
error behaviour (invalid launch -> ValueError, ineligible inputs ->
RuntimeError "... ineligible ...", launch failure -> RuntimeError "...
execution failed").  What differs is the implementation domain: bf16 or fp16
inputs, any batch, head count and sequence length, head_dim 64, computed by
the hand-written kernel in csrc/attention_fwd.hip.

The value tensor may be the reference's head_dim-contiguous view (any key
stride, e.g. the packed QKV view), which the kernel reads as given, or a
seq-contiguous view of a V^T buffer, which it first copies key-major into
its workspace.
"""

from __future__ import annotations

import math

import torch

from ..kernels.hip._library import (
    HipLibraryError,
    check_status,
    dtype_code,
    is_gfx950,
    library_available,
    load_library,
    stream_handle,
)

HIP_STREAMING_DH64_CAUSAL_ATTENTION_BSD_BACKEND = "hip_streaming_dh64_causal_attention_bsd"
_HEAD_DIM = 64
_SUPPORTED_DTYPES = frozenset({torch.bfloat16, torch.float16, torch.float32})
_DEFAULT_BLOCK_M = 128
_DEFAULT_BLOCK_N = 64
_DEFAULT_NUM_WARPS = 4
_DEFAULT_NUM_STAGES = 2
SUPPORTED_BLOCK_M = frozenset({128, 256, 512})
SUPPORTED_BLOCK_N = frozenset({64})
SUPPORTED_NUM_WARPS = frozenset({4, 8})
SUPPORTED_NUM_STAGES = frozenset({1, 2, 3})


def launch_config_is_valid(
    block_m: int,
    block_n: int,
    num_warps: int,
    num_stages: int,
) -> bool:
    """Whether the launch is one the gfx950 kernel implements.

    ``num_warps`` counts 64-wide wavefronts per workgroup (4 or 8) and
    ``num_stages`` the number of LDS tile buffers: 1 or 2 select the plain
    kernel, with 32 or 64 query rows per wavefront (``block_m`` = 32 or 64 x
    ``num_warps``); 3 selects the software-pipelined kernel (4 wavefronts,
    128 rows), in which the score MFMAs of the next tile overlap the
    exponentials of the current one.
    """

    values = (block_m, block_n, num_warps, num_stages)
    return bool(
        not any(isinstance(value, bool) for value in values)
        and all(isinstance(value, int) for value in values)
        and block_m in SUPPORTED_BLOCK_M
        and block_n in SUPPORTED_BLOCK_N
        and num_warps in SUPPORTED_NUM_WARPS
        and num_stages in SUPPORTED_NUM_STAGES
        and (
            # three stages select the software-pipelined kernel (4 waves, 128 rows)
            (block_m == 128 and num_warps == 4)
            if num_stages == 3
            else block_m in (32 * num_warps, 64 * num_warps)
        )
    )


def _validate_launch_config(
    block_m: int, block_n: int, num_warps: int, num_stages: int
) -> None:
    if not launch_config_is_valid(block_m, block_n, num_warps, num_stages):
        raise ValueError("invalid HIP streaming-attention launch configuration")


def _strides(tensor: torch.Tensor) -> tuple[int, ...]:
    """Strides with size-1 axes reported as 0 (they are never stepped).

    A unit stride is kept as is: it names the contiguous axis of the layout.
    """

    return tuple(
        0 if size == 1 and stride != 1 else stride
        for size, stride in zip(tensor.shape, tensor.stride())
    )


def _launch(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    block_m: int,
    block_n: int,
    num_warps: int,
    num_stages: int,
) -> torch.Tensor:
    library = load_library()
    batch, heads, seq_len, head_dim = query.shape
    output = torch.empty(
        (batch, seq_len, heads * head_dim), dtype=query.dtype, device=query.device
    )
    code = dtype_code(query.dtype)
    workspace_bytes = library.sah_causal_attention_workspace_bytes(
        batch, heads, seq_len, head_dim, *_strides(value)[2:], code
    )
    workspace = (
        torch.empty(workspace_bytes, dtype=torch.uint8, device=query.device)
        if workspace_bytes
        else None
    )
    q_strides = _strides(query)
    k_strides = _strides(key)
    v_strides = _strides(value)
    status = library.sah_causal_attention_bsd(
        query.data_ptr(),
        key.data_ptr(),
        value.data_ptr(),
        output.data_ptr(),
        batch,
        heads,
        seq_len,
        head_dim,
        *q_strides[:3],
        *k_strides[:3],
        *v_strides,
        output.stride(0),
        output.stride(1),
        float(scale),
        code,
        block_m,
        block_n,
        num_warps,
        num_stages,
        None if workspace is None else workspace.data_ptr(),
        workspace_bytes,
        stream_handle(query.device),
    )
    check_status(status, "sah_causal_attention_bsd")
    return output


@torch.library.custom_op(
    "shape_aware_hip::streaming_dh64_causal_attention_bsd",
    mutates_args=(),
)
def _streaming_dh64_causal_attention_bsd_op(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    block_m: int,
    block_n: int,
    num_warps: int,
    num_stages: int,
) -> torch.Tensor:
    return _launch(query, key, value, scale, block_m, block_n, num_warps, num_stages)


@_streaming_dh64_causal_attention_bsd_op.register_fake
def _(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    block_m: int,
    block_n: int,
    num_warps: int,
    num_stages: int,
) -> torch.Tensor:
    del key, value, scale, block_m, block_n, num_warps, num_stages
    batch, heads, seq_len, head_dim = query.shape
    return query.new_empty((batch, seq_len, heads * head_dim))


def hip_streaming_dh64_causal_attention_available() -> bool:
    """Whether the gfx950 library loads in this process."""

    return library_available()


def _value_layout_is_supported(value: torch.Tensor) -> bool:
    return value.stride(-1) == 1 or value.stride(-2) == 1


def can_use_hip_streaming_dh64_causal_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_token_mask: torch.Tensor | None = None,
    *,
    causal: bool = True,
    training: bool = False,
    block_m: int = _DEFAULT_BLOCK_M,
    block_n: int = _DEFAULT_BLOCK_N,
    num_warps: int = _DEFAULT_NUM_WARPS,
    num_stages: int = _DEFAULT_NUM_STAGES,
) -> bool:
    """Validate the gfx950 kernel's contract without raising."""

    if not launch_config_is_valid(block_m, block_n, num_warps, num_stages):
        return False
    if training or torch.is_grad_enabled() or not causal:
        return False
    if valid_token_mask is not None or query.device.type != "cuda":
        return False
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        return False
    if query.shape != key.shape or query.shape != value.shape:
        return False
    if query.shape[-1] != _HEAD_DIM or query.shape[2] <= 0 or query.shape[1] <= 0:
        return False
    if query.dtype not in _SUPPORTED_DTYPES:
        return False
    if key.dtype != query.dtype or value.dtype != query.dtype:
        return False
    if query.device != key.device or query.device != value.device:
        return False
    if query.requires_grad or key.requires_grad or value.requires_grad:
        return False
    if query.stride(-1) != 1 or key.stride(-1) != 1:
        return False
    if not _value_layout_is_supported(value):
        return False
    if query.dtype == torch.float32 and value.stride(-1) != 1:
        return False  # the fp32 kernel reads V head_dim-contiguous
    per_16_bytes = 16 // query.element_size()
    for tensor in (query, key, value):
        if tensor.data_ptr() % 16:
            return False
        if any(stride % per_16_bytes for stride in _strides(tensor) if stride != 1):
            return False
    if not hip_streaming_dh64_causal_attention_available():
        return False
    return is_gfx950(query.device)


def prevalidated_hip_streaming_dh64_causal_attention_bsd(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    scale: float | None = None,
    block_m: int = _DEFAULT_BLOCK_M,
    block_n: int = _DEFAULT_BLOCK_N,
    num_warps: int = _DEFAULT_NUM_WARPS,
    num_stages: int = _DEFAULT_NUM_STAGES,
) -> tuple[torch.Tensor, str]:
    """Run the kernel after immutable execution-plan validation."""

    _validate_launch_config(block_m, block_n, num_warps, num_stages)
    resolved_scale = 1.0 / math.sqrt(_HEAD_DIM) if scale is None else float(scale)
    try:
        if torch.compiler.is_compiling():
            output = _streaming_dh64_causal_attention_bsd_op(
                query, key, value, resolved_scale, block_m, block_n, num_warps, num_stages
            )
        else:
            output = _launch(
                query, key, value, resolved_scale, block_m, block_n, num_warps, num_stages
            )
    except (HipLibraryError, RuntimeError, ValueError) as exc:
        raise RuntimeError("HIP streaming attention execution failed") from exc
    return output, HIP_STREAMING_DH64_CAUSAL_ATTENTION_BSD_BACKEND


def hip_streaming_dh64_causal_attention_bsd(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    valid_token_mask: torch.Tensor | None = None,
    *,
    scale: float | None = None,
    causal: bool = True,
    training: bool = False,
    block_m: int = _DEFAULT_BLOCK_M,
    block_n: int = _DEFAULT_BLOCK_N,
    num_warps: int = _DEFAULT_NUM_WARPS,
    num_stages: int = _DEFAULT_NUM_STAGES,
) -> tuple[torch.Tensor, str]:
    """Run the kernel with strict eligibility and no fallback."""

    if not can_use_hip_streaming_dh64_causal_attention(
        query,
        key,
        value,
        valid_token_mask,
        causal=causal,
        training=training,
        block_m=block_m,
        block_n=block_n,
        num_warps=num_warps,
        num_stages=num_stages,
    ):
        raise RuntimeError(
            "HIP streaming attention is ineligible for the requested inputs"
        )
    return prevalidated_hip_streaming_dh64_causal_attention_bsd(
        query,
        key,
        value,
        scale=scale,
        block_m=block_m,
        block_n=block_n,
        num_warps=num_warps,
        num_stages=num_stages,
    )


__all__ = [
    "HIP_STREAMING_DH64_CAUSAL_ATTENTION_BSD_BACKEND",
    "SUPPORTED_BLOCK_M",
    "SUPPORTED_BLOCK_N",
    "SUPPORTED_NUM_STAGES",
    "SUPPORTED_NUM_WARPS",
    "can_use_hip_streaming_dh64_causal_attention",
    "hip_streaming_dh64_causal_attention_available",
    "hip_streaming_dh64_causal_attention_bsd",
    "launch_config_is_valid",
    "prevalidated_hip_streaming_dh64_causal_attention_bsd",
]
