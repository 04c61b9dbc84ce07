"""Immutable execution plans built from typed configurations.

Restates the reference's solution/plan.py:30-341: ``ExecutionContext`` (the
input/model facts that decide legality, with ``with_batch_size`` giving the
inner context of a batch-splitting schedule), ``ExpectedExecutionTrace``
(the path evidence derived from the plan, compared with what forward actually
executed) and ``ExecutionPlan`` (the frozen result of PlanBuilder).  The
dictionaries produced by ``to_dict`` / ``describe`` have the reference's keys.
"""

from __future__ import annotations

from dataclasses import dataclass, fields, replace
from typing import Any

import torch

from .config import (
    AttentionBackend,
    AttentionLaunchParams,
    AttentionOutputBridge,
    AttentionOutputLayout,
    ConfigSpec,
    FFNBackend,
    FFNLaunchParams,
    GemmLaunchParams,
    InitialNormBackend,
    LAUNCHED_ATTENTION_BACKENDS,
    LINEAR_BOUNDARY_RESIDUAL_NORM_BACKENDS,
    NormLaunchParams,
    PrecisionPlan,
    ProjectionBackend,
    QKVLaunchParams,
    QKVMaterialization,
    ResidualNormBackend,
    RuntimeBackend,
)

_LAUNCH_FIELDS = (
    "attention_launch",
    "qkv_launch",
    "attention_output_projection_launch",
    "residual_norm_launch",
    "initial_norm_launch",
    "ffn_launch",
    "ffn_input_launch",
)


def _launch_dict(value: Any) -> dict[str, int] | None:
    return None if value is None else value.to_dict()


@dataclass(frozen=True, slots=True)
class ExecutionContext:
    """Input and model facts that affect plan legality (reference :30-66)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    causal: bool
    device: torch.device
    dtype: torch.dtype
    training: bool
    grad_enabled: bool
    input_contiguous: bool
    has_valid_token_mask: bool
    mask_compatible: bool
    ffn_dim: int | None = None
    num_layers: int | None = None

    @property
    def head_dim(self) -> int | None:
        if self.num_heads <= 0 or self.d_model % self.num_heads:
            return None
        return self.d_model // self.num_heads

    @property
    def dtype_name(self) -> str:
        text = str(self.dtype)
        return text[len("torch."):] if text.startswith("torch.") else text

    @property
    def inference(self) -> bool:
        return not self.training and not self.grad_enabled

    def with_batch_size(self, batch_size: int) -> ExecutionContext:
        """The inner context seen by a batch-splitting schedule."""

        return replace(self, batch_size=batch_size)


@dataclass(frozen=True, slots=True)
class ExpectedExecutionTrace:
    """Path evidence derived from the plan forward consumes (reference :69-185)."""

    runtime_backend: RuntimeBackend
    attention_backend: AttentionBackend
    qkv_projection_backend: ProjectionBackend
    attention_output_projection_backend: ProjectionBackend
    ffn_input_projection_backend: ProjectionBackend
    ffn_output_projection_backend: ProjectionBackend
    precision_plan: PrecisionPlan
    qkv_materialization: QKVMaterialization
    attention_output_bridge: AttentionOutputBridge
    attention_output_layout: AttentionOutputLayout
    ffn_backend: FFNBackend
    residual_norm_backend: ResidualNormBackend
    initial_norm_backend: InitialNormBackend
    attention_compute_dtype: str
    qkv_projection_compute_dtype: str
    attention_output_projection_compute_dtype: str
    ffn_input_projection_compute_dtype: str
    ffn_activation_output_dtype: str
    ffn_output_projection_compute_dtype: str
    attention_calls: int
    qkv_projection_calls: int
    qkv_materialization_calls: int
    attention_output_bridge_calls: int
    attention_output_projection_calls: int
    ffn_calls: int
    ffn_input_projection_calls: int
    ffn_output_projection_calls: int
    residual_norm_calls: int
    initial_norm_calls: int
    runtime_calls: int
    attention_launch: AttentionLaunchParams | None = None
    qkv_launch: QKVLaunchParams | None = None
    attention_output_projection_launch: GemmLaunchParams | None = None
    residual_norm_launch: NormLaunchParams | None = None
    initial_norm_launch: NormLaunchParams | None = None
    ffn_launch: FFNLaunchParams | None = None
    ffn_input_launch: GemmLaunchParams | None = None

    def to_dict(self) -> dict[str, Any]:
        payload: dict[str, Any] = {}
        for item in fields(self):
            value = getattr(self, item.name)
            if item.name in _LAUNCH_FIELDS:
                payload[item.name] = _launch_dict(value)
            elif hasattr(value, "value"):
                payload[item.name] = value.value
            else:
                payload[item.name] = value
        payload["complete"] = True
        return payload


@dataclass(frozen=True, slots=True)
class ExecutionPlan:
    """Strict plan forward executes without hidden fallback (reference :188-341)."""

    config: ConfigSpec
    outer_context: ExecutionContext
    inner_context: ExecutionContext
    attention_backend: AttentionBackend
    attention_compute_dtype: str
    qkv_projection_backend: ProjectionBackend
    qkv_projection_compute_dtype: str
    qkv_materialization: QKVMaterialization
    attention_output_bridge: AttentionOutputBridge
    attention_output_layout: AttentionOutputLayout
    attention_output_projection_backend: ProjectionBackend
    attention_output_projection_compute_dtype: str
    ffn_backend: FFNBackend
    ffn_input_projection_backend: ProjectionBackend
    ffn_input_projection_compute_dtype: str
    ffn_activation_output_dtype: str
    ffn_output_projection_backend: ProjectionBackend
    ffn_output_projection_compute_dtype: str
    precision_plan: PrecisionPlan
    residual_norm_backend: ResidualNormBackend
    initial_norm_backend: InitialNormBackend
    runtime_backend: RuntimeBackend
    compile_mode: str | None
    batch_tile_size: int | None
    microbatch_size: int | None
    reuse_unchanged_input: bool
    attention_launch: AttentionLaunchParams | None
    qkv_launch: QKVLaunchParams | None
    attention_output_projection_launch: GemmLaunchParams | None
    residual_norm_launch: NormLaunchParams | None
    initial_norm_launch: NormLaunchParams | None
    ffn_launch: FFNLaunchParams | None
    ffn_input_launch: GemmLaunchParams | None
    use_d32_residual_norm: bool
    use_masked_residual_norm: bool
    use_masked_initial_norm: bool
    expected_trace: ExpectedExecutionTrace

    @property
    def config_id(self) -> str:
        return self.config.config_id

    @property
    def use_cuda_graph(self) -> bool:
        return self.runtime_backend is RuntimeBackend.CUDA_GRAPH

    @property
    def use_batch_tiled_cuda_graph(self) -> bool:
        return self.runtime_backend is RuntimeBackend.BATCH_TILED_CUDA_GRAPH

    @property
    def use_compiled_forward(self) -> bool:
        return self.runtime_backend is RuntimeBackend.COMPILED_FORWARD

    @property
    def use_streamed_execution(self) -> bool:
        return self.runtime_backend is RuntimeBackend.STREAMED

    @property
    def use_hip_initial_norm(self) -> bool:
        return self.initial_norm_backend is InitialNormBackend.HIP

    @property
    def use_fused_initial_norm_qkv(self) -> bool:
        """Layer 0's LayerNorm runs inside its QKV projection (reference
        :255-256)."""

        return self.initial_norm_backend is InitialNormBackend.HIP_FUSED_QKV

    @property
    def use_fused_mlp_boundary(self) -> bool:
        """The FFN and its residual LayerNorm run as one kernel (reference
        :843-896)."""

        return self.ffn_backend is FFNBackend.HIP_FUSED_MLP_BOUNDARY

    @property
    def use_hip_residual_norm(self) -> bool:
        return self.residual_norm_backend in {
            ResidualNormBackend.HIP_FUSED,
            ResidualNormBackend.HIP_MIXED,
        }

    @property
    def use_linear_boundary_fusion(self) -> bool:
        """The output projections are fused into their residual boundaries
        (reference :259-260)."""

        return self.residual_norm_backend in LINEAR_BOUNDARY_RESIDUAL_NORM_BACKENDS

    @property
    def use_mixed_residual_stream(self) -> bool:
        """fp32 residual stream fed by 16-bit branch outputs."""

        return self.residual_norm_backend in {
            ResidualNormBackend.TRITON_MIXED,
            ResidualNormBackend.HIP_MIXED,
        }

    def describe(self) -> dict[str, Any]:
        """Serialize the plan and its derived evidence (reference :262-341)."""

        if not self.outer_context.causal:
            causal_mask = "none"
        elif self.attention_backend in LAUNCHED_ATTENTION_BACKENDS:
            causal_mask = "online_causal"
        elif self.attention_backend in {
            AttentionBackend.CAUSAL_SDPA,
            AttentionBackend.FP16_CUDNN_SDPA,
            AttentionBackend.FP16_EFFICIENT_SDPA,
        }:
            causal_mask = "implicit_sdpa"
        else:
            causal_mask = "query_block"
        return {
            "config": self.config.to_dict(),
            "qkv_projection": "packed",
            "qkv_projection_backend": self.qkv_projection_backend.value,
            "qkv_projection_compute_dtype": self.qkv_projection_compute_dtype,
            "qkv_materialization": self.qkv_materialization.value,
            "attention_backend": self.attention_backend.value,
            "attention_compute_dtype": self.attention_compute_dtype,
            "attention_output_bridge": self.attention_output_bridge.value,
            "attention_output_layout": self.attention_output_layout.value,
            "attention_output_projection_backend": self.attention_output_projection_backend.value,
            "attention_output_projection_compute_dtype": self.attention_output_projection_compute_dtype,
            "ffn_backend": self.ffn_backend.value,
            "ffn_input_projection_backend": self.ffn_input_projection_backend.value,
            "ffn_input_projection_compute_dtype": self.ffn_input_projection_compute_dtype,
            "ffn_activation_output_dtype": self.ffn_activation_output_dtype,
            "ffn_output_projection_backend": self.ffn_output_projection_backend.value,
            "ffn_output_projection_compute_dtype": self.ffn_output_projection_compute_dtype,
            "precision_plan": self.precision_plan.value,
            "residual_norm_backend": self.residual_norm_backend.value,
            "initial_norm_backend": self.initial_norm_backend.value,
            "runtime_backend": self.runtime_backend.value,
            "compile_mode": self.compile_mode,
            "batch_tile_size": self.batch_tile_size,
            "microbatch_size": self.microbatch_size,
            "reuse_unchanged_input": self.reuse_unchanged_input,
            "use_d32_residual_norm": self.use_d32_residual_norm,
            "use_masked_residual_norm": self.use_masked_residual_norm,
            "use_masked_initial_norm": self.use_masked_initial_norm,
            "qkv_launch": _launch_dict(self.qkv_launch),
            "attention_output_projection_launch": _launch_dict(
                self.attention_output_projection_launch
            ),
            "ffn_launch": _launch_dict(self.ffn_launch),
            "ffn_input_launch": _launch_dict(self.ffn_input_launch),
            "outer_batch_size": self.outer_context.batch_size,
            "inner_batch_size": self.inner_context.batch_size,
            "causal_mask": causal_mask,
            "valid_token_mask": (
                "direct_key_mask" if self.outer_context.has_valid_token_mask else "none"
            ),
        }


__all__ = ["ExecutionContext", "ExecutionPlan", "ExpectedExecutionTrace"]
