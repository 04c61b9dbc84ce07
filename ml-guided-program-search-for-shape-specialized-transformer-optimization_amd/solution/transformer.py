"""Official-compatible Transformer that executes a strict ExecutionPlan.

The plugin contract of the reference (solution/transformer.py:1065-1871):

* ``UserOptimizedTransformer(config)`` with the official constructor and
  ``forward(x, valid_token_mask=None) -> [B, S, D]``;
* ``configure_execution(config=ConfigSpec)``, ``describe_execution_path()``,
  ``set_execution_observation(enabled)``;
* ``copy_model_weights(baseline, optimized, strict=True)``, which packs the
  official q/k/v projections into one ``qkv_proj`` (reference :1806-1871).

Forward resolves a config (an explicit one, an exact deployment-registry
entry, or the platform default), compiles it once per input signature with
PlanBuilder, and executes exactly that plan: every primitive returns a marker
that must equal the planned one (reference :275-288), and an optional
observation records the executed path so it can be compared with the plan's
expected trace (reference :102-238).

On an MI355X (gfx950) the platform default is the HIP program
(``solution.config.hip_config``): hand-written MFMA causal attention writing
[B, S, D] directly, fused residual + LayerNorm kernels at every boundary and
the HIP initial norm; projections and FFN run on hipBLASLt through torch.
Sequences of 32768 tokens or more use the streamed schedule (ordered
microbatches, the final norm of each chunk written straight into the
preallocated output).  If the gfx950 library is missing on a gfx950 device,
config resolution raises instead of quietly running another path.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass, field
from typing import Any

import torch
import torch.nn.functional as F
from torch import nn

from .config import (
    LAUNCHED_ATTENTION_BACKENDS,
    AttentionBackend,
    AttentionOutputBridge,
    AttentionOutputLayout,
    ConfigSpec,
    FFNBackend,
    InitialNormBackend,
    PrecisionPlan,
    ProjectionBackend,
    QKVMaterialization,
    ResidualNormBackend,
    RuntimeBackend,
    hip_config,
    portable_config,
    portable_streamed_config,
)
from .operators import causal_sdpa, reference_causal_attention, residual_add, split_qkv
from .plan import ExecutionContext, ExecutionPlan
from .plan_builder import PlanBuilder

STREAMED_MIN_SEQ_LEN = 32768


def _dtype_name(dtype: torch.dtype) -> str:
    text = str(dtype)
    return text[len("torch."):] if text.startswith("torch.") else text


def _is_official_shape14(config: Any, shape: tuple[int, ...]) -> bool:
    """The reference's one streamed official workload (reference :91-99)."""

    return shape == (32, 100000, 1024) and (
        int(config.num_heads),
        int(config.num_layers),
        int(config.ffn_dim),
        bool(config.causal),
    ) == (16, 2, 1024, True)


def _uses_streamed_scope(config: Any, shape: tuple[int, ...]) -> bool:
    """Long causal sequences run under the streamed schedule.

    Covers the official Shape 14 and any other causal workload of at least
    STREAMED_MIN_SEQ_LEN tokens (e.g. the FFN-4096 long-sequence
    configuration), without fixing the FFN width.
    """

    return _is_official_shape14(config, shape) or (
        len(shape) == 3 and int(shape[1]) >= STREAMED_MIN_SEQ_LEN and bool(config.causal)
    )


# ---------------------------------------------------------------------------
# execution observation


@dataclass(slots=True)
class _ExecutionObservation:
    config_id: str
    runtime_backend: str = RuntimeBackend.EAGER.value
    attention_backends: list[str] = field(default_factory=list)
    residual_norm_backends: list[str] = field(default_factory=list)
    initial_norm_backends: list[str] = field(default_factory=list)
    attention_compute_dtypes: list[str] = field(default_factory=list)
    qkv_projection_backends: list[str] = field(default_factory=list)
    qkv_projection_compute_dtypes: list[str] = field(default_factory=list)
    qkv_materializations: list[str] = field(default_factory=list)
    attention_output_bridges: list[str] = field(default_factory=list)
    attention_output_layouts: list[str] = field(default_factory=list)
    attention_output_projection_backends: list[str] = field(default_factory=list)
    attention_output_projection_compute_dtypes: list[str] = field(default_factory=list)
    ffn_backends: list[str] = field(default_factory=list)
    ffn_input_projection_backends: list[str] = field(default_factory=list)
    ffn_input_projection_compute_dtypes: list[str] = field(default_factory=list)
    ffn_activation_output_dtypes: list[str] = field(default_factory=list)
    ffn_output_projection_backends: list[str] = field(default_factory=list)
    ffn_output_projection_compute_dtypes: list[str] = field(default_factory=list)
    layer_input_dtypes: list[str] = field(default_factory=list)
    layer_output_dtypes: list[str] = field(default_factory=list)
    attention_launches: list[dict[str, int] | None] = field(default_factory=list)
    qkv_launches: list[dict[str, int] | None] = field(default_factory=list)
    attention_output_projection_launches: list[dict[str, int] | None] = field(default_factory=list)
    residual_norm_launches: list[dict[str, int] | None] = field(default_factory=list)
    initial_norm_launches: list[dict[str, int] | None] = field(default_factory=list)
    ffn_launches: list[dict[str, int] | None] = field(default_factory=list)
    ffn_input_launches: list[dict[str, int] | None] = field(default_factory=list)

    # (trace key, list attribute, calls per layer) in the reference's order.
    _PER_LAYER = (
        ("attention_backend", "attention_backends", 1),
        ("qkv_projection_backend", "qkv_projection_backends", 1),
        ("attention_output_projection_backend", "attention_output_projection_backends", 1),
        ("ffn_input_projection_backend", "ffn_input_projection_backends", 1),
        ("ffn_output_projection_backend", "ffn_output_projection_backends", 1),
        ("qkv_materialization", "qkv_materializations", 1),
        ("attention_output_bridge", "attention_output_bridges", 1),
        ("attention_output_layout", "attention_output_layouts", 1),
        ("ffn_backend", "ffn_backends", 1),
        ("residual_norm_backend", "residual_norm_backends", 2),
        ("attention_compute_dtype", "attention_compute_dtypes", 1),
        ("qkv_projection_compute_dtype", "qkv_projection_compute_dtypes", 1),
        ("attention_output_projection_compute_dtype", "attention_output_projection_compute_dtypes", 1),
        ("ffn_input_projection_compute_dtype", "ffn_input_projection_compute_dtypes", 1),
        ("ffn_activation_output_dtype", "ffn_activation_output_dtypes", 1),
        ("ffn_output_projection_compute_dtype", "ffn_output_projection_compute_dtypes", 1),
    )
    _LAUNCHES = (
        ("attention_launch", "attention_launches", 1),
        ("qkv_launch", "qkv_launches", 1),
        ("attention_output_projection_launch", "attention_output_projection_launches", 1),
        ("residual_norm_launch", "residual_norm_launches", 2),
        ("ffn_launch", "ffn_launches", 1),
        ("ffn_input_launch", "ffn_input_launches", 1),
    )

    @staticmethod
    def _uniform(values: list[Any]) -> Any | None:
        if not values:
            return None
        first = values[0]
        return first if all(value == first for value in values) else None

    def describe(self, expected_layers: int) -> dict[str, Any]:
        initial_calls = 1 if expected_layers else 0
        complete = all(
            len(getattr(self, attr)) == per * expected_layers
            for _, attr, per in self._PER_LAYER + self._LAUNCHES
        )
        complete = complete and len(self.layer_input_dtypes) == expected_layers
        complete = complete and len(self.layer_output_dtypes) == expected_layers
        complete = complete and len(self.initial_norm_backends) == initial_calls
        complete = complete and len(self.initial_norm_launches) == initial_calls
        precision_plan = _infer_precision_plan(
            self._uniform(self.qkv_projection_backends),
            self._uniform(self.attention_output_projection_backends),
            self._uniform(self.ffn_input_projection_backends),
            self._uniform(self.ffn_output_projection_backends),
        )
        complete = complete and precision_plan is not None
        payload: dict[str, Any] = {
            "config_id": self.config_id,
            "runtime_backend": self.runtime_backend,
        }
        for key, attr, _ in self._PER_LAYER[:5]:
            payload[key] = self._uniform(getattr(self, attr))
        payload["precision_plan"] = precision_plan
        for key, attr, _ in self._PER_LAYER[5:]:
            payload[key] = self._uniform(getattr(self, attr))
        payload["initial_norm_backend"] = self._uniform(self.initial_norm_backends)
        payload.update(
            attention_calls=len(self.attention_backends),
            qkv_projection_calls=len(self.qkv_projection_backends),
            qkv_materialization_calls=len(self.qkv_materializations),
            attention_output_bridge_calls=len(self.attention_output_bridges),
            attention_output_projection_calls=len(self.attention_output_projection_backends),
            ffn_calls=len(self.ffn_backends),
            ffn_input_projection_calls=len(self.ffn_input_projection_backends),
            ffn_output_projection_calls=len(self.ffn_output_projection_backends),
            residual_norm_calls=len(self.residual_norm_backends),
            initial_norm_calls=len(self.initial_norm_backends),
            runtime_calls=1,
        )
        for key, attr, _ in self._LAUNCHES:
            payload[key] = self._uniform(getattr(self, attr))
        payload["initial_norm_launch"] = self._uniform(self.initial_norm_launches)
        payload["complete"] = complete
        return payload


def _infer_precision_plan(
    qkv: str | None, attention_output: str | None, ffn_input: str | None, ffn_output: str | None
) -> str | None:
    fp16 = {ProjectionBackend.AUTOCAST_FP16.value, ProjectionBackend.FP16_SHADOW.value}
    mask = tuple(item in fp16 for item in (qkv, attention_output, ffn_input, ffn_output))
    plans = {
        (False, False, False, False): PrecisionPlan.INPUT_DTYPE,
        (True, False, False, False): PrecisionPlan.FP16_QKV_ATTENTION,
        (True, True, False, False): PrecisionPlan.FP16_ATTENTION_BRANCH,
        (False, False, True, False): PrecisionPlan.FP16_FFN_INPUT_FP32_GELU,
        (True, True, True, False): PrecisionPlan.FP16_ATTENTION_AND_FFN_INPUT,
        (False, False, True, True): PrecisionPlan.FP16_FFN_BRANCH,
        (False, False, False, True): PrecisionPlan.FP16_FFN_OUTPUT,
        (True, True, True, True): PrecisionPlan.FP16_CORE,
    }
    plan = plans.get(mask)
    return None if plan is None else plan.value


def _strict_backend_marker(actual: str, *, expected_marker: str, planned_backend: str) -> str:
    """A primitive's marker must be the planned one (reference :275-288)."""

    if actual != expected_marker:
        raise RuntimeError(
            "execution backend marker does not match the compiled plan: "
            f"expected marker {expected_marker!r}, received {actual!r}"
        )
    return planned_backend


def _launch_dict(value: Any) -> dict[str, int] | None:
    return None if value is None else value.to_dict()


# ---------------------------------------------------------------------------
# modules


class _FP16ShadowLinear(nn.Linear):
    """Linear layer with optional non-persistent FP16 inference weights
    (reference :291-353)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True) -> None:
        super().__init__(in_features, out_features, bias=bias)
        self.register_buffer("_fp16_shadow_weight", None, persistent=False)
        self.register_buffer("_fp16_shadow_bias", None, persistent=False)

    def materialize_fp16_shadow(self) -> None:
        if self._fp16_shadow_weight is not None:
            return
        self._fp16_shadow_weight = self.weight.detach().to(torch.float16).contiguous()
        self._fp16_shadow_bias = (
            None if self.bias is None else self.bias.detach().to(torch.float16).contiguous()
        )

    def clear_fp16_shadow(self) -> None:
        self._fp16_shadow_weight = None
        self._fp16_shadow_bias = None

    def forward_backend(self, value: torch.Tensor, backend: ProjectionBackend) -> torch.Tensor:
        if backend is ProjectionBackend.INPUT_DTYPE:
            if value.dtype != self.weight.dtype:
                value = value.to(self.weight.dtype)
            return self(value)
        if backend is ProjectionBackend.AUTOCAST_FP16:
            with torch.autocast(device_type=value.device.type, dtype=torch.float16, enabled=True):
                return self(value)
        if backend is ProjectionBackend.FP16_SHADOW:
            weight = self._fp16_shadow_weight
            if weight is None:
                raise RuntimeError("FP16 shadow weights must be materialized before use")
            return F.linear(value.to(torch.float16), weight, self._fp16_shadow_bias)
        raise AssertionError(f"unhandled projection backend: {backend}")


class _SelfAttention(nn.Module):
    """Packed QKV projection followed by the planned causal attention."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim**-0.5
        self.qkv_proj = _FP16ShadowLinear(d_model, 3 * d_model, bias=True)
        self.out_proj = _FP16ShadowLinear(d_model, d_model, bias=True)

    def forward(
        self,
        value: torch.Tensor,
        valid_token_mask: torch.Tensor | None,
        causal: bool,
        plan: ExecutionPlan,
        observation: _ExecutionObservation | None,
        *,
        project: bool = True,
        initial_norm: nn.LayerNorm | None = None,
    ) -> torch.Tensor:
        """The attention branch.  With ``project=False`` (the linear-boundary
        plans, reference :620-726) it returns the [B, S, D] context before the
        output projection, which the fused boundary multiplies.  With
        ``initial_norm`` (layer 0 of a fused initial-norm plan, reference
        :1419-1423) ``value`` is the un-normalized input and the LayerNorm runs
        inside the QKV projection."""

        batch, seq, _ = value.shape
        backend = plan.attention_backend
        if initial_norm is not None and plan.qkv_materialization is not QKVMaterialization.HIP_NATIVE_BHSD:
            raise RuntimeError("the fused initial norm needs the HIP native-layout QKV projection")
        if plan.qkv_materialization is QKVMaterialization.HIP_NATIVE_BHSD:
            # The reference's native-layout branch (solution/transformer.py:384-431):
            # the projection kernel writes head-major Q / K / V itself, V as
            # [B, H, S, 64], which the HIP attention reads as given.
            from .kernels.projection.hip_qkv_layout import (
                HIP_INITIAL_NORM_QKV_BACKEND,
                HIP_QKV_NATIVE_BHSD_BACKEND,
                prevalidated_hip_initial_norm_qkv_native_bhsd,
                prevalidated_hip_qkv_native_bhsd,
            )

            launch = plan.qkv_launch
            if launch is None:
                raise RuntimeError("HIP native-layout QKV plan is missing launch parameters")
            launch_args = dict(
                num_heads=self.num_heads,
                block_m=launch.block_m,
                block_n=launch.block_n,
                block_k=launch.block_k,
                num_warps=launch.num_warps,
                value_layout="bhsd",
            )
            if initial_norm is None:
                query, key, projected, marker = prevalidated_hip_qkv_native_bhsd(
                    value, self.qkv_proj.weight, self.qkv_proj.bias, **launch_args
                )
                expected = HIP_QKV_NATIVE_BHSD_BACKEND
            else:
                query, key, projected, marker = prevalidated_hip_initial_norm_qkv_native_bhsd(
                    value, initial_norm, self.qkv_proj.weight, self.qkv_proj.bias, **launch_args
                )
                expected = HIP_INITIAL_NORM_QKV_BACKEND
            _strict_backend_marker(
                marker,
                expected_marker=expected,
                planned_backend=plan.qkv_materialization.value,
            )
            qkv_dtype = query.dtype
            if observation is not None:
                observation.qkv_materializations.append(plan.qkv_materialization.value)
                observation.qkv_launches.append(_launch_dict(plan.qkv_launch))
        else:
            packed = self.qkv_proj.forward_backend(value, plan.qkv_projection_backend)
            qkv_dtype = packed.dtype
            query, key, projected = split_qkv(
                packed,
                self.num_heads,
                contiguous=plan.qkv_materialization is QKVMaterialization.CONTIGUOUS,
            )
            if observation is not None:
                storage = packed.untyped_storage().data_ptr()
                shares = all(t.untyped_storage().data_ptr() == storage for t in (query, key, projected))
                actual = QKVMaterialization.VIEW if shares else QKVMaterialization.CONTIGUOUS
                if actual is not plan.qkv_materialization:
                    raise RuntimeError("QKV materialization does not match the plan")
                observation.qkv_materializations.append(actual.value)
                observation.qkv_launches.append(_launch_dict(plan.qkv_launch))

        if backend is AttentionBackend.HIP_STREAMING_DH64:
            from .shape14.hip_streaming_dh64 import (
                HIP_STREAMING_DH64_CAUSAL_ATTENTION_BSD_BACKEND,
                prevalidated_hip_streaming_dh64_causal_attention_bsd,
            )

            launch = plan.attention_launch
            if launch is None:
                raise RuntimeError("HIP streaming attention plan is missing launch parameters")
            context, marker = prevalidated_hip_streaming_dh64_causal_attention_bsd(
                query,
                key,
                projected,
                scale=self.scale,
                block_m=launch.block_m,
                block_n=launch.block_n,
                num_warps=launch.num_warps,
                num_stages=launch.num_stages,
            )
            actual_backend = _strict_backend_marker(
                marker,
                expected_marker=HIP_STREAMING_DH64_CAUSAL_ATTENTION_BSD_BACKEND,
                planned_backend=backend.value,
            )
        elif backend is AttentionBackend.CAUSAL_SDPA:
            context = causal_sdpa(
                query, key, projected, valid_token_mask, scale=self.scale, causal=causal
            )
            actual_backend = backend.value
        elif backend is AttentionBackend.REFERENCE_STREAMING:
            context = reference_causal_attention(
                query, key, projected, valid_token_mask, scale=self.scale, causal=causal
            )
            actual_backend = backend.value
        else:
            raise RuntimeError(f"attention backend {backend.value} is not executable here")

        layout = AttentionOutputLayout.BHSD if context.ndim == 4 else AttentionOutputLayout.BSD
        if layout is not plan.attention_output_layout:
            raise RuntimeError("attention output layout does not match the plan")
        if plan.attention_output_bridge is AttentionOutputBridge.TORCH_BHSD_TO_BSD:
            context = context.transpose(1, 2).contiguous().view(batch, seq, self.d_model)
        elif plan.attention_output_bridge is not AttentionOutputBridge.ATTENTION_DIRECT_BSD:
            raise RuntimeError(
                f"attention bridge {plan.attention_output_bridge.value} is not executable here"
            )
        output = (
            self.out_proj.forward_backend(context, plan.attention_output_projection_backend)
            if project
            else context
        )
        if observation is not None:
            observation.attention_backends.append(actual_backend)
            observation.attention_compute_dtypes.append(
                "float16"
                if backend in LAUNCHED_ATTENTION_BACKENDS and query.dtype == torch.float16
                else _dtype_name(query.dtype)
            )
            observation.qkv_projection_backends.append(plan.qkv_projection_backend.value)
            observation.qkv_projection_compute_dtypes.append(_dtype_name(qkv_dtype))
            observation.attention_output_layouts.append(layout.value)
            observation.attention_output_bridges.append(plan.attention_output_bridge.value)
            observation.attention_output_projection_backends.append(
                plan.attention_output_projection_backend.value
            )
            observation.attention_output_projection_compute_dtypes.append(
                _dtype_name(output.dtype if project else value.dtype)
            )
            observation.attention_output_projection_launches.append(
                _launch_dict(plan.attention_output_projection_launch)
            )
            observation.attention_launches.append(_launch_dict(plan.attention_launch))
        if not project:
            return output
        if output.dtype != value.dtype and not plan.use_mixed_residual_stream:
            output = output.to(value.dtype)
        if valid_token_mask is not None:
            output.masked_fill_(~valid_token_mask[..., None], 0)
        return output


class _TransformerBlock(nn.Module):
    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = _SelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = _FP16ShadowLinear(d_model, ffn_dim)
        self.ffn_out = _FP16ShadowLinear(ffn_dim, d_model)

    def attention_update(
        self,
        normalized: torch.Tensor,
        valid_token_mask: torch.Tensor | None,
        causal: bool,
        plan: ExecutionPlan,
        observation: _ExecutionObservation | None,
        *,
        project: bool = True,
        initial_norm: nn.LayerNorm | None = None,
    ) -> torch.Tensor:
        return self.attention(
            normalized, valid_token_mask, causal, plan, observation, project=project, initial_norm=initial_norm
        )

    def ffn_update(
        self,
        normalized: torch.Tensor,
        plan: ExecutionPlan,
        observation: _ExecutionObservation | None,
        *,
        project: bool = True,
    ) -> torch.Tensor:
        """Exact-GELU FFN (reference :816-1062): the TORCH branch, the
        elementwise Exact-GELU kernel after the input projection (reference
        :945-965, here the gfx950 kernel), or the fused Linear + bias + exact
        GELU input projection (reference :898-935, here the gfx950 kernel);
        then the output projection.  With ``project=False`` (the
        linear-boundary plans, reference :1001-1033) it returns the hidden
        activation, which the fused boundary multiplies."""

        if plan.ffn_backend is FFNBackend.HIP_LINEAR_EXACT_GELU:
            from .kernels.ffn.hip_linear_gelu import (
                HIP_LINEAR_EXACT_GELU_BACKEND,
                prevalidated_hip_linear_exact_gelu,
            )

            launch = plan.ffn_input_launch
            if launch is None:
                raise RuntimeError("HIP Linear + Exact-GELU plan is missing launch parameters")
            hidden, marker = prevalidated_hip_linear_exact_gelu(
                normalized,
                self.ffn_in.weight,
                self.ffn_in.bias,
                block_m=launch.block_m,
                block_n=launch.block_n,
                block_k=launch.block_k,
                num_warps=launch.num_warps,
                num_stages=launch.num_stages,
            )
            _strict_backend_marker(
                marker,
                expected_marker=HIP_LINEAR_EXACT_GELU_BACKEND,
                planned_backend=plan.ffn_backend.value,
            )
            input_compute_dtype = _dtype_name(hidden.dtype)
        elif plan.ffn_backend is FFNBackend.HIP_EXACT_GELU:
            from .kernels.ffn.hip_exact_gelu import HIP_EXACT_GELU_BACKEND, prevalidated_hip_exact_gelu

            launch = plan.ffn_launch
            if launch is None:
                raise RuntimeError("HIP Exact-GELU plan is missing launch parameters")
            projected = self.ffn_in.forward_backend(normalized, plan.ffn_input_projection_backend)
            input_compute_dtype = _dtype_name(projected.dtype)
            # in place: the projection is a temporary of this block
            hidden, marker = prevalidated_hip_exact_gelu(
                projected, block_size=launch.block_size, num_warps=launch.num_warps, out=projected
            )
            _strict_backend_marker(
                marker, expected_marker=HIP_EXACT_GELU_BACKEND, planned_backend=plan.ffn_backend.value
            )
        else:
            projected = self.ffn_in.forward_backend(normalized, plan.ffn_input_projection_backend)
            input_compute_dtype = _dtype_name(projected.dtype)
            if plan.ffn_activation_output_dtype == "float32":
                projected = projected.float()
            hidden = F.gelu(projected, approximate="none")
        update = (
            self.ffn_out.forward_backend(hidden, plan.ffn_output_projection_backend) if project else hidden
        )
        if observation is not None:
            observation.ffn_input_projection_backends.append(plan.ffn_input_projection_backend.value)
            observation.ffn_input_projection_compute_dtypes.append(input_compute_dtype)
            observation.ffn_activation_output_dtypes.append(_dtype_name(hidden.dtype))
            observation.ffn_output_projection_backends.append(plan.ffn_output_projection_backend.value)
            observation.ffn_output_projection_compute_dtypes.append(
                _dtype_name(update.dtype if project else normalized.dtype)
            )
            observation.ffn_launches.append(_launch_dict(plan.ffn_launch))
            observation.ffn_input_launches.append(_launch_dict(plan.ffn_input_launch))
            observation.ffn_backends.append(plan.ffn_backend.value)
        if not project:
            return update
        if update.dtype != normalized.dtype and not plan.use_mixed_residual_stream:
            update = update.to(normalized.dtype)
        return update


    def mlp_boundary(
        self,
        normalized: torch.Tensor,
        value: torch.Tensor,
        next_norm: nn.LayerNorm,
        plan: ExecutionPlan,
        observation: _ExecutionObservation | None,
        *,
        out: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """The whole FFN and the residual LayerNorm after it in one kernel
        (reference: the TRITON_FUSED_MLP_BOUNDARY branch,
        solution/transformer.py:843-896, here the gfx950 kernel); neither the
        hidden activation nor the update reaches HBM."""

        from .kernels.boundary.hip_mlp_residual_norm import (
            HIP_MLP_RESIDUAL_NORM_BACKEND,
            hip_mlp_residual_norm,
        )

        launch = plan.residual_norm_launch
        if launch is None:
            raise RuntimeError("fused MLP boundary is missing launch parameters")
        destination = (
            out if out is not None and out.dtype == value.dtype and out.is_contiguous() else None
        )
        value, normalized, marker = hip_mlp_residual_norm(
            normalized,
            self.ffn_in.weight,
            self.ffn_in.bias,
            self.ffn_out.weight,
            self.ffn_out.bias,
            value,
            next_norm,
            block_rows=launch.block_rows,
            num_warps=launch.num_warps,
            out=destination,
        )
        _strict_backend_marker(
            marker,
            expected_marker=HIP_MLP_RESIDUAL_NORM_BACKEND,
            planned_backend=plan.ffn_backend.value,
        )
        if observation is not None:
            dtype = _dtype_name(value.dtype)
            observation.ffn_input_projection_backends.append(plan.ffn_input_projection_backend.value)
            observation.ffn_input_projection_compute_dtypes.append(dtype)
            observation.ffn_activation_output_dtypes.append(dtype)
            observation.ffn_output_projection_backends.append(plan.ffn_output_projection_backend.value)
            observation.ffn_output_projection_compute_dtypes.append(dtype)
            observation.ffn_launches.append(None)
            observation.ffn_input_launches.append(None)
            observation.ffn_backends.append(plan.ffn_backend.value)
            # the FFN boundary's residual norm runs inside the fused kernel
            observation.residual_norm_backends.append(plan.residual_norm_backend.value)
            observation.residual_norm_launches.append(_launch_dict(plan.residual_norm_launch))
        return value, normalized


class UserOptimizedTransformer(nn.Module):
    """Solution entry with the official constructor and forward API."""

    def __init__(self, config: Any) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            [
                _TransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
                for _ in range(config.num_layers)
            ]
        )
        self.final_norm = nn.LayerNorm(config.d_model)
        self._graph_replay: Any = None  # GraphReplay of the cuda_graph runtime
        self._runtime_plan_signature: tuple[object, ...] | None = None
        self._runtime_plan: ExecutionPlan | None = None
        self._execution_observation_enabled = False
        self._last_execution_observation: dict[str, Any] | None = None
        self._classified_mask: torch.Tensor | None = None
        self._classified_mask_version: int | None = None
        self._classified_mask_is_all_valid = False
        self._plan_builder = PlanBuilder()
        self._explicit_config: ConfigSpec | None = None
        self._active_config = portable_config()
        self._deployment_signature: tuple[object, ...] | None = None

    # ------------------------------------------------------------ state
    def _invalidate_runtime_state(self) -> None:
        self._graph_replay = None
        self._runtime_plan_signature = None
        self._runtime_plan = None
        self._last_execution_observation = None
        self._classified_mask = None
        self._classified_mask_version = None
        self._classified_mask_is_all_valid = False

    def _apply(self, function: Any, recurse: bool = True) -> UserOptimizedTransformer:
        result = super()._apply(function, recurse=recurse)
        self._clear_fp16_shadow_weights()
        self._invalidate_runtime_state()
        self._deployment_signature = None
        if self._explicit_config is None and next(self.parameters()).is_cuda:
            self._resolve_default_config()
        return result

    def _materialize_fp16_shadow_weights(self, plan: ExecutionPlan) -> None:
        for layer in self.layers:
            for backend, module in (
                (plan.qkv_projection_backend, layer.attention.qkv_proj),
                (plan.attention_output_projection_backend, layer.attention.out_proj),
                (plan.ffn_input_projection_backend, layer.ffn_in),
                (plan.ffn_output_projection_backend, layer.ffn_out),
            ):
                if backend is ProjectionBackend.FP16_SHADOW:
                    module.materialize_fp16_shadow()

    def _clear_fp16_shadow_weights(self) -> None:
        for module in self.modules():
            if isinstance(module, _FP16ShadowLinear):
                module.clear_fp16_shadow()

    # ----------------------------------------------------------- configs
    def _platform_default(self, shape: tuple[int, ...], device: torch.device) -> ConfigSpec:
        streamed = _uses_streamed_scope(self.config, shape)
        if device.type == "cuda":
            from .kernels.hip._library import is_gfx950, load_library

            if is_gfx950(device):
                load_library()  # a gfx950 device without the library is an error
                if streamed:
                    from .shape14.defaults import DEFAULT_MICROBATCH_SIZE, hip_streamed_config

                    batch = int(shape[0])
                    microbatch = DEFAULT_MICROBATCH_SIZE if batch % DEFAULT_MICROBATCH_SIZE == 0 else 1
                    return hip_streamed_config(microbatch_size=microbatch)
                return hip_config()
        return portable_streamed_config() if streamed else portable_config()

    def _resolve_default_config(self, value: torch.Tensor | None = None) -> None:
        """Exact deployed config, else the platform default, else portable."""

        if self._explicit_config is not None:
            return
        parameter = next(self.parameters())
        device = parameter.device if value is None else value.device
        dtype = parameter.dtype if value is None else value.dtype
        shape = (
            (self.config.batch_size, self.config.seq_len, self.config.d_model)
            if value is None
            else tuple(value.shape)
        )
        signature = (
            device.type,
            device.index,
            dtype,
            shape,
            torch.get_float32_matmul_precision(),
            self.training,
            value is not None and torch.is_grad_enabled(),
        )
        if signature == self._deployment_signature:
            return
        context = self._execution_context(value)
        selected: ConfigSpec | None = None
        if device.type == "cuda":
            selected = self._deployed_config(device, dtype, shape)
            if selected is not None and not self._plan_builder.evaluate(selected, context).accepted:
                selected = None
            if selected is None:
                candidate = self._platform_default(shape, device)
                if self._plan_builder.evaluate(candidate, context).accepted:
                    selected = candidate
        if selected is None:
            selected = (
                portable_streamed_config()
                if _uses_streamed_scope(self.config, shape)
                else portable_config()
            )
        if selected != self._active_config:
            self._invalidate_runtime_state()
        self._active_config = selected
        self._deployment_signature = signature

    def _deployed_config(
        self, device: torch.device, dtype: torch.dtype, shape: tuple[int, ...]
    ) -> ConfigSpec | None:
        from deployment.environment import EnvironmentFingerprint, ImplementationScope
        from deployment.registry import ShapeFingerprint, resolve_deployed_config

        scope = (
            ImplementationScope.SHAPE14
            if _uses_streamed_scope(self.config, shape)
            else ImplementationScope.RESIDENT
        )
        try:
            hardware = EnvironmentFingerprint.detect(device, scope=scope)
        except (RuntimeError, ValueError):
            return None
        deployed_shape = ShapeFingerprint(
            batch_size=int(shape[0]),
            qkv_dim=int(self.config.d_model),
            heads=int(self.config.num_heads),
            seq_len=int(shape[1]),
            layers=int(self.config.num_layers),
            causal=bool(self.config.causal),
            ffn_dim=int(self.config.ffn_dim),
            dtype=_dtype_name(dtype),
            padding_ratio=0.0,
            input_scale=1.0,
        )
        return resolve_deployed_config(hardware=hardware, shape=deployed_shape)

    def configure_execution(self, *, config: ConfigSpec) -> None:
        """Install one explicit config after strict compilation for this model."""

        if not isinstance(config, ConfigSpec):
            raise TypeError("config must be ConfigSpec")
        self._plan_builder.build(config, self._execution_context())
        self._invalidate_runtime_state()
        self._explicit_config = config
        self._active_config = config
        self._deployment_signature = None

    def _execution_context(
        self,
        value: torch.Tensor | None = None,
        valid_token_mask: torch.Tensor | None = None,
    ) -> ExecutionContext:
        parameter = next(self.parameters())
        if value is None:
            device, dtype = parameter.device, parameter.dtype
            shape = (self.config.batch_size, self.config.seq_len, self.config.d_model)
            contiguous, has_mask, mask_ok, grad = True, False, True, False
        else:
            device, dtype, shape = value.device, value.dtype, tuple(value.shape)
            contiguous = value.is_contiguous()
            has_mask = valid_token_mask is not None
            mask_ok = valid_token_mask is None or (
                valid_token_mask.device == value.device
                and valid_token_mask.dtype == torch.bool
                and valid_token_mask.ndim == 2
                and tuple(valid_token_mask.shape) == tuple(value.shape[:2])
            )
            grad = torch.is_grad_enabled()
        return ExecutionContext(
            batch_size=shape[0],
            seq_len=shape[1],
            d_model=shape[-1],
            num_heads=self.config.num_heads,
            causal=bool(self.config.causal),
            device=device,
            dtype=dtype,
            training=self.training,
            grad_enabled=grad,
            input_contiguous=contiguous,
            has_valid_token_mask=has_mask,
            mask_compatible=mask_ok,
            ffn_dim=self.config.ffn_dim,
            num_layers=self.config.num_layers,
        )

    def _execution_plan(
        self, value: torch.Tensor | None = None, valid_token_mask: torch.Tensor | None = None
    ) -> ExecutionPlan:
        return self._plan_builder.build(
            self._active_config, self._execution_context(value, valid_token_mask)
        )

    def _cached_execution_plan(
        self, value: torch.Tensor, valid_token_mask: torch.Tensor | None
    ) -> ExecutionPlan:
        mask_signature = None
        if valid_token_mask is not None:
            mask_signature = (
                valid_token_mask.device,
                valid_token_mask.dtype,
                tuple(valid_token_mask.shape),
            )
        # The active config object itself (compared by identity first, by
        # value otherwise): its config_id is a SHA-256 of its canonical JSON,
        # too slow to form on every call.
        signature = (
            self._active_config,
            value.device,
            value.dtype,
            tuple(value.shape),
            value.is_contiguous(),
            mask_signature,
            self.training,
            torch.is_grad_enabled(),
        )
        if signature != self._runtime_plan_signature:
            self._runtime_plan = self._execution_plan(value, valid_token_mask)
            self._runtime_plan_signature = signature
        assert self._runtime_plan is not None
        return self._runtime_plan

    def describe_execution_path(self) -> dict[str, Any]:
        plan = self._runtime_plan or self._execution_plan()
        description = plan.describe()
        expected = plan.expected_trace.to_dict()
        expected["config_id"] = plan.config_id
        description.update(
            requested_config_id=self._active_config.config_id,
            planned_config_id=plan.config_id,
            runtime_backend=plan.runtime_backend.value,
            expected_execution_signature=expected,
            observed_execution_signature=self._last_execution_observation,
        )
        return description

    def set_execution_observation(self, enabled: bool) -> None:
        self._execution_observation_enabled = bool(enabled)
        if enabled:
            self._last_execution_observation = None

    # ---------------------------------------------------------- execution
    def _initial_norm(
        self,
        value: torch.Tensor,
        plan: ExecutionPlan,
        observation: _ExecutionObservation | None,
    ) -> torch.Tensor:
        norm = self.layers[0].norm1
        branch_dtype = torch.float16 if plan.use_mixed_residual_stream else value.dtype
        if plan.use_fused_initial_norm_qkv:
            # layer 0's QKV projection normalizes (reference :1364-1371)
            normalized = value
        elif plan.initial_norm_backend is InitialNormBackend.HIP:
            from .kernels.norm.hip_residual import HIP_LAYER_NORM_BACKEND, hip_layer_norm

            launch = plan.initial_norm_launch
            if launch is None:
                raise RuntimeError("HIP initial norm plan is missing launch parameters")
            normalized, marker = hip_layer_norm(
                value,
                norm,
                normalized_dtype=branch_dtype,
                block_rows=launch.block_rows,
                num_warps=launch.num_warps,
            )
            _strict_backend_marker(
                marker,
                expected_marker=HIP_LAYER_NORM_BACKEND,
                planned_backend=plan.initial_norm_backend.value,
            )
        elif plan.initial_norm_backend is InitialNormBackend.TORCH:
            normalized = norm(value)
            if normalized.dtype != branch_dtype:
                normalized = normalized.to(branch_dtype)
        else:
            raise RuntimeError(
                f"initial norm {plan.initial_norm_backend.value} is not executable here"
            )
        if observation is not None:
            observation.initial_norm_backends.append(plan.initial_norm_backend.value)
            observation.initial_norm_launches.append(_launch_dict(plan.initial_norm_launch))
        return normalized

    def _forward_eager(
        self,
        value: torch.Tensor,
        valid_token_mask: torch.Tensor | None,
        plan: ExecutionPlan,
        *,
        out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """One (micro)batch through every layer (reference :1346-1513).

        ``out``, when given, receives the final normalized output (used by
        the streamed driver to write each chunk into the logical output).
        """

        observation = (
            _ExecutionObservation(config_id=plan.config_id)
            if self._execution_observation_enabled and not torch.compiler.is_compiling()
            else None
        )
        if not self.layers:
            return self.final_norm(value)
        normalized = self._initial_norm(value, plan, observation)
        causal = bool(self.config.causal)
        fused = plan.use_linear_boundary_fusion
        for index, layer in enumerate(self.layers):
            if observation is not None:
                observation.layer_input_dtypes.append(_dtype_name(value.dtype))
            last = index + 1 == len(self.layers)
            next_norm = self.final_norm if last else self.layers[index + 1].norm1
            initial_norm = layer.norm1 if index == 0 and plan.use_fused_initial_norm_qkv else None
            if fused:
                context = layer.attention_update(
                    normalized, valid_token_mask, causal, plan, observation, project=False, initial_norm=initial_norm
                )
                value, normalized = self._apply_linear_boundary(
                    context, layer.attention.out_proj, value, layer.norm2, plan, observation
                )
                hidden = layer.ffn_update(normalized, plan, observation, project=False)
                value, normalized = self._apply_linear_boundary(
                    hidden, layer.ffn_out, value, next_norm, plan, observation, out=out if last else None
                )
            else:
                update = layer.attention_update(
                    normalized, valid_token_mask, causal, plan, observation, initial_norm=initial_norm
                )
                value, normalized = self._apply_residual_norm(
                    value, update, layer.norm2, valid_token_mask, plan, observation, final_boundary=False
                )
                if plan.use_fused_mlp_boundary:
                    value, normalized = layer.mlp_boundary(
                        normalized, value, next_norm, plan, observation, out=out if last else None
                    )
                else:
                    update = layer.ffn_update(normalized, plan, observation)
                    value, normalized = self._apply_residual_norm(
                        value,
                        update,
                        next_norm,
                        valid_token_mask,
                        plan,
                        observation,
                        final_boundary=last,
                        out=out if last else None,
                    )
            if observation is not None:
                observation.layer_output_dtypes.append(_dtype_name(normalized.dtype))
        if valid_token_mask is not None:
            normalized.masked_fill_(~valid_token_mask[..., None], 0)
        if observation is not None:
            self._last_execution_observation = observation.describe(len(self.layers))
        return normalized

    @staticmethod
    def _apply_linear_boundary(
        source: torch.Tensor,
        linear: _FP16ShadowLinear,
        value: torch.Tensor,
        layer_norm: nn.LayerNorm,
        plan: ExecutionPlan,
        observation: _ExecutionObservation | None,
        *,
        out: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """A branch's output projection fused with the residual add and the
        LayerNorm after it (reference: the triton_linear_residual_norm calls,
        solution/transformer.py:699-725 and :1001-1033, here the gfx950
        kernel); the update never reaches HBM."""

        from .kernels.boundary.hip_linear_residual_norm import (
            HIP_LINEAR_RESIDUAL_NORM_BACKEND,
            hip_linear_residual_norm,
        )

        if plan.residual_norm_backend is not ResidualNormBackend.HIP_LINEAR_FUSED:
            raise RuntimeError(f"linear boundary {plan.residual_norm_backend.value} is not executable here")
        launch = plan.residual_norm_launch
        if launch is None:
            raise RuntimeError("HIP linear boundary plan is missing launch parameters")
        destination = (
            out if out is not None and out.dtype == value.dtype and out.is_contiguous() else None
        )
        value, normalized, marker = hip_linear_residual_norm(
            source,
            linear.weight,
            linear.bias,
            value,
            layer_norm,
            block_rows=launch.block_rows,
            num_warps=launch.num_warps,
            out=destination,
        )
        actual = _strict_backend_marker(
            marker,
            expected_marker=HIP_LINEAR_RESIDUAL_NORM_BACKEND,
            planned_backend=plan.residual_norm_backend.value,
        )
        if observation is not None:
            observation.residual_norm_backends.append(actual)
            observation.residual_norm_launches.append(_launch_dict(plan.residual_norm_launch))
        return value, normalized

    @staticmethod
    def _apply_residual_norm(
        value: torch.Tensor,
        update: torch.Tensor,
        layer_norm: nn.LayerNorm,
        valid_token_mask: torch.Tensor | None,
        plan: ExecutionPlan,
        observation: _ExecutionObservation | None,
        *,
        final_boundary: bool,
        out: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """One residual boundary and the LayerNorm after it (reference :1515-1644)."""

        backend = plan.residual_norm_backend
        if backend in {ResidualNormBackend.HIP_FUSED, ResidualNormBackend.HIP_MIXED}:
            from .kernels.norm.hip_residual import (
                HIP_RESIDUAL_LAYER_NORM_BACKEND,
                hip_residual_layer_norm,
            )

            launch = plan.residual_norm_launch
            if launch is None:
                raise RuntimeError("HIP residual norm plan is missing launch parameters")
            if backend is ResidualNormBackend.HIP_MIXED:
                normalized_dtype = torch.float32 if final_boundary else torch.float16
            else:
                normalized_dtype = value.dtype
            destination = (
                out if out is not None and out.dtype == normalized_dtype and out.is_contiguous() else None
            )
            value, normalized, marker = hip_residual_layer_norm(
                value,
                update,
                layer_norm,
                normalized_dtype=normalized_dtype,
                block_rows=launch.block_rows,
                num_warps=launch.num_warps,
                out=destination,
            )
            actual = _strict_backend_marker(
                marker,
                expected_marker=HIP_RESIDUAL_LAYER_NORM_BACKEND,
                planned_backend=backend.value,
            )
        elif backend is ResidualNormBackend.TORCH:
            value = residual_add(value, update, valid_token_mask)
            normalized = layer_norm(value)
            actual = backend.value
        else:
            raise RuntimeError(f"residual norm {backend.value} is not executable here")
        if observation is not None:
            observation.residual_norm_backends.append(actual)
            observation.residual_norm_launches.append(_launch_dict(plan.residual_norm_launch))
        return value, normalized

    def _effective_valid_token_mask(
        self, value: torch.Tensor, valid_token_mask: torch.Tensor | None
    ) -> torch.Tensor | None:
        """Collapse an unchanged all-valid mask to None (reference :1646-1675)."""

        if valid_token_mask is None or torch.compiler.is_compiling():
            return valid_token_mask
        if not (
            valid_token_mask.device == value.device
            and valid_token_mask.dtype == torch.bool
            and valid_token_mask.ndim == 2
            and tuple(valid_token_mask.shape) == tuple(value.shape[:2])
        ):
            return valid_token_mask
        try:
            version = valid_token_mask._version
        except RuntimeError:
            return None if bool(valid_token_mask.all().item()) else valid_token_mask
        if self._classified_mask is not valid_token_mask or self._classified_mask_version != version:
            self._classified_mask = valid_token_mask
            self._classified_mask_version = version
            self._classified_mask_is_all_valid = bool(valid_token_mask.all().item())
        return None if self._classified_mask_is_all_valid else valid_token_mask

    def forward(
        self, x: torch.Tensor, valid_token_mask: torch.Tensor | None = None
    ) -> torch.Tensor:
        if torch.compiler.is_compiling():
            if self._active_config.schedule.runtime not in {RuntimeBackend.EAGER, RuntimeBackend.STREAMED}:
                raise RuntimeError("a Solution-owned runtime cannot run under torch.compile")
            valid_token_mask = self._effective_valid_token_mask(x, valid_token_mask)
            plan = self._execution_plan(x, valid_token_mask)
        else:
            self._resolve_default_config(x)
            valid_token_mask = self._effective_valid_token_mask(x, valid_token_mask)
            plan = self._cached_execution_plan(x, valid_token_mask)
        if ProjectionBackend.FP16_SHADOW in (
            plan.qkv_projection_backend,
            plan.attention_output_projection_backend,
            plan.ffn_input_projection_backend,
            plan.ffn_output_projection_backend,
        ):
            self._materialize_fp16_shadow_weights(plan)
        if plan.use_streamed_execution:
            microbatch = plan.microbatch_size
            if microbatch is None or microbatch <= 0:
                raise RuntimeError("streamed plan is missing its microbatch size")
            from .shape14.executor import execute_streamed

            output = execute_streamed(
                x,
                valid_token_mask,
                microbatch_size=microbatch,
                forward_chunk=lambda chunk, mask, destination: self._forward_eager(
                    chunk, mask, plan, out=destination
                ),
                write_into_output=True,
            )
            if self._execution_observation_enabled and self._last_execution_observation is not None:
                self._last_execution_observation["runtime_backend"] = RuntimeBackend.STREAMED.value
            return output
        if plan.use_cuda_graph:
            if self._graph_replay is None:
                from .runtimes.graph_replay import GraphReplay

                self._graph_replay = GraphReplay(reuse_unchanged_input=plan.reuse_unchanged_input)
            output = self._graph_replay.run(
                lambda value, mask: self._forward_eager(value, mask, plan), x, valid_token_mask
            )
            if self._execution_observation_enabled and self._last_execution_observation is not None:
                self._last_execution_observation["runtime_backend"] = RuntimeBackend.CUDA_GRAPH.value
            return output
        if plan.runtime_backend is not RuntimeBackend.EAGER:
            raise RuntimeError(f"runtime {plan.runtime_backend.value} is not executable here")
        return self._forward_eager(x, valid_token_mask, plan)


# ---------------------------------------------------------------------------
# weight mapping


def _packed_source_keys(target_key: str) -> tuple[str, str, str] | None:
    marker = ".attention.qkv_proj."
    if marker not in target_key:
        return None
    prefix, suffix = target_key.split(marker, maxsplit=1)
    return tuple(
        f"{prefix}.attention.{projection}.{suffix}" for projection in ("q_proj", "k_proj", "v_proj")
    )  # type: ignore[return-value]


def copy_model_weights(baseline: nn.Module, optimized: nn.Module, strict: bool = True) -> None:
    """Copy official weights; pack q/k/v into qkv_proj (reference :1806-1871)."""

    source = baseline.state_dict()
    target = optimized.state_dict()
    mapped: dict[str, torch.Tensor] = {}
    consumed: set[str] = set()
    for key, tensor in target.items():
        packed_keys = _packed_source_keys(key)
        if packed_keys is None:
            if key in source:
                mapped[key] = source[key]
                consumed.add(key)
            continue
        if not all(name in source for name in packed_keys):
            continue
        packed = torch.cat([source[name] for name in packed_keys], dim=0)
        if packed.shape != tensor.shape:
            raise RuntimeError(
                f"packed tensor shape mismatch for {key}: "
                f"source={tuple(packed.shape)}, target={tuple(tensor.shape)}"
            )
        mapped[key] = packed
        consumed.update(packed_keys)
    missing = sorted(set(target) - set(mapped))
    unused = sorted(set(source) - consumed)
    if strict and (missing or unused):
        raise RuntimeError(
            "strict weight mapping failed; "
            f"missing target keys={missing}, unused source keys={unused}"
        )
    incompatible = optimized.load_state_dict(mapped, strict=strict)
    clear = getattr(optimized, "_clear_fp16_shadow_weights", None)
    if callable(clear):
        clear()
    if not strict:
        parts = []
        if missing or incompatible.missing_keys:
            parts.append(f"missing target keys={sorted(set(missing + incompatible.missing_keys))}")
        if unused:
            parts.append(f"unused source keys={unused}")
        if incompatible.unexpected_keys:
            parts.append(f"unexpected mapped keys={sorted(incompatible.unexpected_keys)}")
        if parts:
            warnings.warn("non-strict weight mapping: " + ", ".join(parts), RuntimeWarning, stacklevel=2)


__all__ = ["UserOptimizedTransformer", "copy_model_weights"]
