"""Plan validation for the streamed schedule and the gfx950 streaming attention.

validate_streamed_runtime restates the reference's rule
(solution/shape14/planning.py:13-41): no token mask, the microbatch must not
exceed and must divide the logical batch, and the inner context is the outer
one with batch = microbatch.

validate_hip_streaming_attention replaces the reference's Triton rule
(solution/shape14/planning.py:54-108).  The reference admits only the exact
official Shape 14 (B1/2/4 microbatch, L2, H16, S100000, D1024, F1024) with
FP16 QKV; the gfx950 kernel is shape-general, so the rule is what the kernel
needs: head_dim 64, 16-bit (bf16 or fp16) QKV, a gfx950 device with the
library loaded, and a launch the kernel implements.
"""

from __future__ import annotations

from collections.abc import Callable

from ..config import ConfigSpec
from ..plan import ExecutionContext

Reject = Callable[[str, str, str], None]


def validate_streamed_runtime(
    config: ConfigSpec,
    context: ExecutionContext,
    reject: Reject,
) -> ExecutionContext:
    """Validate the streamed outer schedule and return its inner context."""

    microbatch_size = config.schedule.microbatch_size
    if microbatch_size is None:
        raise RuntimeError("streamed configuration is missing its microbatch size")
    if context.has_valid_token_mask:
        reject(
            "mask_not_supported",
            "schedule.runtime",
            "streamed execution currently requires an all-valid workload",
        )
    if microbatch_size > context.batch_size:
        reject(
            "microbatch_exceeds_batch",
            "schedule.microbatch_size",
            "microbatch cannot exceed the logical batch",
        )
    elif context.batch_size % microbatch_size:
        reject(
            "microbatch_not_divisor",
            "schedule.microbatch_size",
            "microbatch must divide the logical batch",
        )
    return context.with_batch_size(microbatch_size)


def _hip_attention_available(capability: bool | None) -> bool:
    if capability is not None:
        return capability
    from .hip_streaming_dh64 import hip_streaming_dh64_causal_attention_available

    return hip_streaming_dh64_causal_attention_available()


def validate_hip_streaming_attention(
    *,
    config: ConfigSpec,
    context: ExecutionContext,
    capability: bool | None,
    gcn_arch: str | None,
    qkv_dtype: str,
    reject: Reject,
) -> None:
    """Validate the gfx950 streaming attention for one (inner) context."""

    if not _hip_attention_available(capability):
        reject(
            "backend_unavailable",
            "program.attention",
            "the gfx950 HIP streaming attention library is not loaded",
        )
    if gcn_arch != "gfx950":
        reject(
            "requires_gfx950",
            "program.attention",
            "HIP streaming attention requires an MI355X (gfx950) GPU",
        )
    if context.head_dim != 64:
        reject(
            "unsupported_shape",
            "program.attention",
            "HIP streaming attention is specialized for head_dim 64",
        )
    if qkv_dtype not in {"bfloat16", "float16", "float32"}:
        reject(
            "unsupported_dtype",
            "program.qkv_projection",
            "HIP streaming attention supports BF16, FP16 and FP32 QKV",
        )
    launch = config.schedule.attention_launch
    if launch is None:
        raise RuntimeError("HIP streaming attention is missing launch parameters")
    from .hip_streaming_dh64 import launch_config_is_valid

    if not launch_config_is_valid(
        launch.block_m, launch.block_n, launch.num_warps, launch.num_stages
    ):
        reject(
            "unsupported_launch_value",
            "schedule.attention_launch",
            "HIP streaming launch is outside the implemented kernel",
        )


__all__ = ["validate_hip_streaming_attention", "validate_streamed_runtime"]
