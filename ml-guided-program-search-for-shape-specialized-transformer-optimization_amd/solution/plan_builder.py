"""Static legality compiler: ConfigSpec + ExecutionContext -> ExecutionPlan.

Restates the reference's PlanBuilder (solution/plan_builder.py:52-263,
:294-1392): a non-throwing ``evaluate`` that collects structured
``ConstraintViolation``s (code, field, message) and a strict ``build`` that
raises ``ConfigRejectedError``; no policy lookup and no substitution of another
configuration.  ``HardwareCapabilities`` is an injectable snapshot, so tests
can evaluate legality without a GPU.

Backends of this build: the reference's portable PyTorch primitives
(reference-order and SDPA attention, view/contiguous QKV, the torch bridge,
torch FFN and norms, eager and streamed runtimes) plus the gfx950 kernels
(HIP streaming attention, HIP fused/mixed residual norm, HIP initial norm).
The reference's Triton/cuDNN kernels, torch.compile paths and CUDA-graph
runtimes are not part of the gfx950 build; their configs still parse and are
rejected here with ``backend_unavailable``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch

from .config import (
    DIRECT_BSD_ATTENTION_BACKENDS,
    TRITON_ATTENTION_BACKENDS,
    AttentionBackend,
    AttentionOutputBridge,
    ConfigSpec,
    FFNBackend,
    InitialNormBackend,
    PrecisionPlan,
    ProjectionBackend,
    QKVMaterialization,
    ResidualNormBackend,
    RuntimeBackend,
)
from .plan import ExecutionContext, ExecutionPlan, ExpectedExecutionTrace

Reject = Callable[[str, str, str], None]
_FP16_PROJECTIONS = frozenset({ProjectionBackend.AUTOCAST_FP16, ProjectionBackend.FP16_SHADOW})


@dataclass(frozen=True, slots=True)
class ConstraintViolation:
    """One statically known reason a configuration cannot execute."""

    code: str
    field: str
    message: str

    def to_dict(self) -> dict[str, str]:
        return {"code": self.code, "field": self.field, "message": self.message}


@dataclass(frozen=True, slots=True)
class CompileRejection:
    config_id: str
    violations: tuple[ConstraintViolation, ...]

    def __post_init__(self) -> None:
        if not self.violations:
            raise ValueError("CompileRejection requires at least one violation")

    def to_dict(self) -> dict[str, Any]:
        return {
            "config_id": self.config_id,
            "violations": [violation.to_dict() for violation in self.violations],
        }


class ConfigRejectedError(ValueError):
    """Raised by strict compilation of an illegal configuration."""

    def __init__(self, rejection: CompileRejection) -> None:
        self.rejection = rejection
        summary = "; ".join(f"{item.field}:{item.code}" for item in rejection.violations)
        super().__init__(f"configuration {rejection.config_id} rejected: {summary}")


@dataclass(frozen=True, slots=True)
class CompilationResult:
    config_id: str
    plan: ExecutionPlan | None
    rejection: CompileRejection | None

    def __post_init__(self) -> None:
        if (self.plan is None) == (self.rejection is None):
            raise ValueError("exactly one of plan and rejection must be present")

    @property
    def accepted(self) -> bool:
        return self.plan is not None

    @property
    def violations(self) -> tuple[ConstraintViolation, ...]:
        return () if self.rejection is None else self.rejection.violations

    def require_plan(self) -> ExecutionPlan:
        if self.plan is not None:
            return self.plan
        assert self.rejection is not None
        raise ConfigRejectedError(self.rejection)


@dataclass(frozen=True, slots=True)
class HardwareCapabilities:
    """Injectable hardware/backend snapshot (reference :124-200 plus HIP facts).

    ``gcn_arch`` is the ROCm architecture name ("gfx950" on MI355X); the
    ``hip_*`` flags say whether the gfx950 library loads.  Every ``triton_*``
    flag is False in this build (no Triton kernels).
    """

    device_type: str
    compute_capability: tuple[int, int] | None
    shared_memory_per_block: int | None
    mem_efficient_sdp: bool
    cudnn_sdp: bool
    cudnn_available: bool
    torch_compile: bool
    triton_shape13_attention: bool
    triton_dh8_attention: bool
    triton_residual_norm: bool
    triton_mixed_residual_norm: bool
    triton_initial_norm: bool
    triton_exact_gelu: bool
    triton_streaming_dh64_attention: bool | None = None
    triton_qkv_native_bhsd: bool = False
    triton_attention_output_projection: bool = False
    triton_linear_exact_gelu: bool = False
    triton_d32_residual_norm: bool = False
    triton_masked_norm: bool = False
    triton_linear_residual_norm: bool = False
    triton_fused_ffn_residual_norm: bool = False
    gcn_arch: str | None = None
    hip_streaming_dh64_attention: bool | None = None
    hip_residual_norm: bool = False
    hip_initial_norm: bool = False
    hip_linear_exact_gelu: bool = False
    hip_exact_gelu: bool = False
    hip_qkv_native_bhsd: bool = False
    hip_linear_residual_norm: bool = False
    hip_mlp_residual_norm: bool = False

    @property
    def is_gfx950(self) -> bool:
        return self.gcn_arch == "gfx950"

    @classmethod
    def detect(cls, device: torch.device) -> HardwareCapabilities:
        device_type = device.type
        compute_capability = None
        shared_memory = None
        gcn_arch = None
        hip_available = False
        if device_type == "cuda" and torch.cuda.is_available():
            index = device.index if device.index is not None else torch.cuda.current_device()
            compute_capability = torch.cuda.get_device_capability(index)
            properties = torch.cuda.get_device_properties(index)
            shared_memory = int(
                getattr(properties, "shared_memory_per_block_optin", 0)
                or getattr(properties, "shared_memory_per_block", 0)
                or 0
            ) or None
            arch = getattr(properties, "gcnArchName", None)
            gcn_arch = None if arch is None else str(arch).split(":")[0]
            if gcn_arch == "gfx950":
                from .kernels.hip._library import library_available

                hip_available = library_available()
        return cls(
            device_type=device_type,
            compute_capability=compute_capability,
            shared_memory_per_block=shared_memory,
            mem_efficient_sdp=False,
            cudnn_sdp=False,
            cudnn_available=False,
            torch_compile=False,
            triton_shape13_attention=False,
            triton_dh8_attention=False,
            triton_residual_norm=False,
            triton_mixed_residual_norm=False,
            triton_initial_norm=False,
            triton_exact_gelu=False,
            triton_streaming_dh64_attention=False,
            gcn_arch=gcn_arch,
            hip_streaming_dh64_attention=hip_available,
            hip_residual_norm=hip_available,
            hip_initial_norm=hip_available,
            hip_linear_exact_gelu=hip_available,
            hip_exact_gelu=hip_available,
            hip_qkv_native_bhsd=hip_available,
            hip_linear_residual_norm=hip_available,
            hip_mlp_residual_norm=hip_available,
        )


def _unavailable(reject: Reject, field: str, what: str) -> None:
    reject("backend_unavailable", field, f"{what} is not part of the gfx950 build")


class PlanBuilder:
    """Build exactly one execution plan, or reject it with reasons."""

    def evaluate(
        self,
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities | None = None,
    ) -> CompilationResult:
        if not isinstance(config, ConfigSpec):
            raise TypeError("config must be ConfigSpec")
        if not isinstance(context, ExecutionContext):
            raise TypeError("context must be ExecutionContext")
        capabilities = hardware or HardwareCapabilities.detect(context.device)
        violations: list[ConstraintViolation] = []

        def reject(code: str, field: str, message: str) -> None:
            violations.append(ConstraintViolation(code, field, message))

        self._validate_context(context, capabilities, reject)
        inner = self._validate_runtime(config, context, capabilities, reject)
        self._validate_projections(config, inner, reject)
        self._validate_qkv_materialization(config, inner, capabilities, reject)
        self._validate_attention(config, inner, capabilities, reject)
        self._validate_attention_bridge(config, inner, capabilities, reject)
        self._validate_ffn(config, inner, capabilities, reject)
        self._validate_residual_norm(config, inner, capabilities, reject)
        self._validate_initial_norm(config, inner, capabilities, reject)
        if violations:
            rejection = CompileRejection(config.config_id, tuple(violations))
            return CompilationResult(config.config_id, None, rejection)
        return CompilationResult(
            config.config_id, self._build_plan(config, context, inner, capabilities), None
        )

    def build(
        self,
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities | None = None,
    ) -> ExecutionPlan:
        """Build a plan or raise; never substitute another configuration."""

        return self.evaluate(config, context, hardware).require_plan()

    # ------------------------------------------------------------------ context
    @staticmethod
    def _validate_context(
        context: ExecutionContext, hardware: HardwareCapabilities, reject: Reject
    ) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads"):
            value = getattr(context, name)
            if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
                reject("non_positive", name, f"{name} must be positive")
        if context.num_heads > 0 and context.d_model % context.num_heads:
            reject("not_divisible", "num_heads", "d_model must be divisible by num_heads")
        if context.has_valid_token_mask and not context.mask_compatible:
            reject(
                "incompatible_mask",
                "valid_token_mask",
                "token mask does not match the input shape, device, or dtype",
            )
        if hardware.device_type != context.device.type:
            reject(
                "device_mismatch",
                "hardware.device_type",
                "hardware capabilities do not describe the input device",
            )

    # ------------------------------------------------------------------ runtime
    @staticmethod
    def _validate_runtime(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> ExecutionContext:
        runtime = config.schedule.runtime
        if runtime is RuntimeBackend.EAGER:
            return context
        if context.device.type != "cuda":
            reject("requires_cuda", "schedule.runtime", "runtime requires a GPU")
        if not context.inference:
            reject("requires_inference", "schedule.runtime", "runtime is available only for inference")
        if not context.input_contiguous:
            reject("requires_contiguous_input", "schedule.runtime", "runtime requires a contiguous input")
        if runtime is RuntimeBackend.STREAMED:
            from .shape14.planning import validate_streamed_runtime

            return validate_streamed_runtime(config, context, reject)
        if runtime is RuntimeBackend.CUDA_GRAPH:  # a HIP graph on ROCm
            return context
        _unavailable(reject, "schedule.runtime", f"the {runtime.value} runtime")
        if runtime is RuntimeBackend.BATCH_TILED_CUDA_GRAPH:
            tile = config.schedule.batch_tile_size
            assert tile is not None
            return context.with_batch_size(tile)
        return context

    # -------------------------------------------------------------- projections
    @staticmethod
    def _validate_projections(
        config: ConfigSpec, context: ExecutionContext, reject: Reject
    ) -> None:
        for name in (
            "qkv_projection",
            "attention_output_projection",
            "ffn_input_projection",
            "ffn_output_projection",
        ):
            if getattr(config.program, name) is ProjectionBackend.INPUT_DTYPE:
                continue
            if context.device.type != "cuda":
                reject("requires_cuda", f"program.{name}", "FP16 projection requires a GPU")
            if not context.inference:
                reject(
                    "requires_inference",
                    f"program.{name}",
                    "FP16 projection is available only for inference",
                )

    @staticmethod
    def _validate_qkv_materialization(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        materialization = config.program.qkv_materialization
        if materialization is QKVMaterialization.TRITON_NATIVE_BHSD:
            _unavailable(reject, "program.qkv_materialization", "Triton native-layout QKV projection")
            return
        if materialization is not QKVMaterialization.HIP_NATIVE_BHSD:
            return
        # The reference's TRITON_NATIVE_BHSD branch (solution/plan_builder.py:381-446)
        # for 16-bit models with native-dtype weights and this kernel's shapes.
        from .kernels.projection.hip_qkv_layout import launch_config_is_valid, supported_shape

        field = "program.qkv_materialization"
        if not hardware.hip_qkv_native_bhsd:
            reject("backend_unavailable", field, "the gfx950 HIP library is not loaded")
        if context.device.type != "cuda" or not hardware.is_gfx950:
            reject("requires_gfx950", field, "HIP kernels require an MI355X (gfx950) GPU")
        if not context.inference:
            reject("requires_inference", field, "native BHSD QKV is available only for inference")
        if context.dtype not in {torch.float16, torch.bfloat16}:
            reject("unsupported_dtype", field, "HIP native BHSD QKV runs on FP16 and BF16 models")
        if config.program.qkv_projection is not ProjectionBackend.INPUT_DTYPE:
            reject(
                "backend_incompatible",
                "program.qkv_projection",
                "HIP native BHSD QKV multiplies the native-dtype packed weights",
            )
        if not supported_shape(context.d_model, context.num_heads):
            reject(
                "unsupported_shape",
                field,
                "HIP native BHSD QKV needs d_model % 256 == 0 and head_dim % 8 == 0",
            )
        if context.batch_size * context.seq_len >= 2**31:
            reject("unsupported_shape", field, "HIP native BHSD QKV needs batch * seq_len < 2^31")
        if config.schedule.runtime is RuntimeBackend.COMPILED_FORWARD:
            reject(
                "runtime_incompatible",
                "schedule.runtime",
                "native BHSD QKV is not nested in compiled forward",
            )
        launch = config.schedule.qkv_launch
        assert launch is not None
        if not launch_config_is_valid(launch.block_m, launch.block_n, launch.block_k, launch.num_warps):
            reject(
                "unsupported_launch_value",
                "schedule.qkv_launch",
                "HIP native BHSD QKV implements (256, 256, 64, 8)",
            )

    # ---------------------------------------------------------------- attention
    @staticmethod
    def _validate_attention(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        backend = config.program.attention
        qkv_dtype = PlanBuilder._projection_dtype(config.program.qkv_projection, context)
        if backend is AttentionBackend.REFERENCE_STREAMING:
            if context.dtype not in {torch.float16, torch.bfloat16, torch.float32}:
                reject(
                    "unsupported_dtype",
                    "program.attention",
                    "reference attention supports FP16, BF16, and FP32",
                )
            return
        if backend is AttentionBackend.CAUSAL_SDPA:
            if qkv_dtype not in {"float16", "float32"}:
                reject(
                    "comparator_unsafe_dtype",
                    "program.attention",
                    "native SDPA is excluded for BF16 comparator safety",
                )
            return
        if not context.inference:
            reject(
                "requires_inference",
                "program.attention",
                "selected attention backend is available only for inference",
            )
        if not context.causal:
            reject("requires_causal", "program.attention", "selected attention backend implements causal attention")
        if context.device.type != "cuda":
            reject("requires_cuda", "program.attention", "backend requires a GPU")
        if context.has_valid_token_mask:
            reject("mask_not_supported", "program.attention", "backend does not accept a token mask")
        if backend is AttentionBackend.HIP_STREAMING_DH64:
            from .shape14.planning import validate_hip_streaming_attention

            validate_hip_streaming_attention(
                config=config,
                context=context,
                capability=hardware.hip_streaming_dh64_attention,
                gcn_arch=hardware.gcn_arch,
                qkv_dtype=qkv_dtype,
                reject=reject,
            )
            return
        names = {
            AttentionBackend.FP16_EFFICIENT_SDPA: "forced memory-efficient FP16 SDPA",
            AttentionBackend.FP16_CUDNN_SDPA: "cuDNN SDPA",
        }
        if backend in names:
            _unavailable(reject, "program.attention", names[backend])
            return
        if backend in TRITON_ATTENTION_BACKENDS:
            _unavailable(reject, "program.attention", f"Triton attention {backend.value}")
            return
        raise AssertionError(f"unhandled attention backend: {backend}")

    @staticmethod
    def _validate_attention_bridge(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        backend = config.program.attention
        bridge = config.program.attention_output_bridge
        if bridge is AttentionOutputBridge.ATTENTION_DIRECT_BSD:
            if backend not in DIRECT_BSD_ATTENTION_BACKENDS:
                reject(
                    "backend_incompatible",
                    "program.attention_output_bridge",
                    "direct BSD output is implemented only by the tiled attention kernels",
                )
            return
        if backend in {
            AttentionBackend.TRITON_DH8,
            AttentionBackend.TRITON_STREAMING_DH64,
            AttentionBackend.HIP_STREAMING_DH64,
        }:
            reject(
                "backend_incompatible",
                "program.attention_output_bridge",
                "selected attention produces BSD directly",
            )
        if bridge is AttentionOutputBridge.TRITON_BHSD_PROJECTION:
            _unavailable(reject, "program.attention_output_bridge", "Triton BHSD output projection")

    # ---------------------------------------------------------------------- FFN
    @staticmethod
    def _validate_ffn(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        backend = config.program.ffn
        if backend is FFNBackend.TORCH:
            return
        if backend is FFNBackend.HIP_EXACT_GELU:
            # The elementwise activation of the reference's TRITON_EXACT_GELU
            # branch (solution/plan_builder.py:870-900), for 16-bit models.
            from .kernels.ffn.hip_exact_gelu import launch_config_is_valid as gelu_launch_is_valid

            field = "program.ffn"
            _validate_hip_common(context, hardware, hardware.hip_exact_gelu, field, reject)
            if context.dtype not in {torch.float16, torch.bfloat16}:
                reject("unsupported_dtype", field, "HIP Exact-GELU runs on FP16 and BF16 models")
            if config.program.ffn_input_projection is not ProjectionBackend.INPUT_DTYPE:
                reject(
                    "backend_incompatible",
                    "program.ffn_input_projection",
                    "HIP Exact-GELU activates the model-dtype projection in place",
                )
            if config.program.precision_plan is not PrecisionPlan.INPUT_DTYPE:
                reject(
                    "backend_incompatible",
                    "program.precision_plan",
                    "HIP Exact-GELU writes the activation in the model dtype",
                )
            ffn_launch = config.schedule.ffn_launch
            assert ffn_launch is not None
            if not gelu_launch_is_valid(ffn_launch.block_size, ffn_launch.num_warps):
                reject(
                    "unsupported_launch_value",
                    "schedule.ffn_launch",
                    "HIP Exact-GELU needs block_size = 512 x num_warps x {1, 2, 4, 8}",
                )
            return
        if backend is FFNBackend.HIP_LINEAR_EXACT_GELU:
            # The fused input projection of the reference's
            # TRITON_LINEAR_EXACT_GELU branch (solution/plan_builder.py:825-866),
            # for 16-bit models with native-dtype weights.
            from .kernels.ffn.hip_linear_gelu import launch_config_is_valid, supported_features

            field = "program.ffn"
            _validate_hip_common(context, hardware, hardware.hip_linear_exact_gelu, field, reject)
            if context.dtype not in {torch.float16, torch.bfloat16}:
                reject("unsupported_dtype", field, "HIP Linear + Exact-GELU runs on FP16 and BF16 models")
            if config.program.ffn_input_projection is not ProjectionBackend.INPUT_DTYPE:
                reject(
                    "backend_incompatible",
                    "program.ffn_input_projection",
                    "HIP Linear + Exact-GELU multiplies the native-dtype input weights",
                )
            if config.program.precision_plan is not PrecisionPlan.INPUT_DTYPE:
                reject(
                    "backend_incompatible",
                    "program.precision_plan",
                    "HIP Linear + Exact-GELU writes the activation in the model dtype",
                )
            if context.ffn_dim is None or not supported_features(context.d_model, context.ffn_dim):
                reject(
                    "unsupported_shape",
                    field,
                    "HIP Linear + Exact-GELU needs d_model % 64 == 0 and ffn_dim % 256 == 0",
                )
            launch = config.schedule.ffn_input_launch
            assert launch is not None
            if not launch_config_is_valid(
                launch.block_m, launch.block_n, launch.block_k, launch.num_warps, launch.num_stages
            ):
                reject(
                    "unsupported_launch_value",
                    "schedule.ffn_input_launch",
                    "HIP Linear + Exact-GELU implements (256, 256, 64, 8, 2)",
                )
            return
        if backend is FFNBackend.HIP_FUSED_MLP_BOUNDARY:
            PlanBuilder._validate_fused_mlp_boundary(config, context, hardware, reject)
            return
        what = "torch.compile FFN" if backend is FFNBackend.COMPILED else f"Triton FFN {backend.value}"
        _unavailable(reject, "program.ffn", what)

    @staticmethod
    def _validate_fused_mlp_boundary(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        """The reference's TRITON_FUSED_MLP_BOUNDARY rules (solution/
        plan_builder.py:783-800): the kernel's widths, native-dtype FFN
        weights, the launch carried by residual_norm_launch.  The reference
        pairs it with its fused linear boundary at the attention output; here
        the pair is the fused residual norm (HIP_FUSED), because the HIP
        linear boundary has no kernel at these widths."""

        from .kernels.boundary.hip_mlp_residual_norm import launch_config_is_valid, supported_shape

        field = "program.ffn"
        _validate_hip_common(context, hardware, hardware.hip_mlp_residual_norm, field, reject)
        if context.dtype not in {torch.float16, torch.bfloat16}:
            reject("unsupported_dtype", field, "the fused MLP boundary runs on FP16 and BF16 models")
        if context.ffn_dim is None or not supported_shape(context.d_model, context.ffn_dim):
            reject(
                "unsupported_shape",
                field,
                "the fused MLP boundary supports d_model 128 and 256 with ffn_dim % 64 == 0",
            )
        for name in ("ffn_input_projection", "ffn_output_projection"):
            if getattr(config.program, name) is not ProjectionBackend.INPUT_DTYPE:
                reject(
                    "backend_incompatible",
                    f"program.{name}",
                    "the fused MLP boundary multiplies the native-dtype FFN weights",
                )
        if config.program.precision_plan is not PrecisionPlan.INPUT_DTYPE:
            reject(
                "backend_incompatible",
                "program.precision_plan",
                "the fused MLP boundary keeps the hidden activation in the model dtype",
            )
        if config.program.residual_norm is not ResidualNormBackend.HIP_FUSED:
            reject(
                "backend_incompatible",
                "program.residual_norm",
                "the fused MLP boundary pairs with the HIP fused residual norm",
            )
        if config.schedule.runtime is RuntimeBackend.COMPILED_FORWARD:
            reject("runtime_incompatible", "schedule.runtime", "the fused MLP boundary is not nested in compiled forward")
        launch = config.schedule.residual_norm_launch
        if launch is None or not launch_config_is_valid(context.d_model, launch.block_rows, launch.num_warps):
            reject(
                "unsupported_launch_value",
                "schedule.residual_norm_launch",
                "the fused MLP boundary runs 64 rows per workgroup of 4 wavefronts",
            )

    # ------------------------------------------------------------ residual norm
    @staticmethod
    def _validate_residual_norm(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        backend = config.program.residual_norm
        if backend is ResidualNormBackend.TORCH:
            return
        if backend is ResidualNormBackend.HIP_LINEAR_FUSED:
            PlanBuilder._validate_linear_boundary(config, context, hardware, reject)
            return
        if backend not in {ResidualNormBackend.HIP_FUSED, ResidualNormBackend.HIP_MIXED}:
            what = (
                "torch.compile residual norm"
                if backend is ResidualNormBackend.COMPILED
                else f"Triton residual norm {backend.value}"
            )
            _unavailable(reject, "program.residual_norm", what)
            return
        from .kernels.norm.hip_residual import launch_config_is_valid, supported_width

        field = "program.residual_norm"
        _validate_hip_common(context, hardware, hardware.hip_residual_norm, field, reject)
        launch = config.schedule.residual_norm_launch
        assert launch is not None
        if not launch_config_is_valid(launch.block_rows, launch.num_warps):
            reject(
                "unsupported_launch_value",
                "schedule.residual_norm_launch",
                "HIP norm needs block_rows a multiple of num_warps and at most 64",
            )
        if backend is ResidualNormBackend.HIP_FUSED:
            if context.dtype not in {torch.float32, torch.float16, torch.bfloat16}:
                reject("unsupported_dtype", field, "HIP fused norm supports FP32, FP16 and BF16 streams")
            elif not supported_width(context.d_model, context.dtype):
                reject("unsupported_shape", field, "HIP fused norm has no kernel for this width")
            return
        # HIP_MIXED: fp32 stream, FP16 branch outputs (the reference's mixed boundary).
        if context.dtype != torch.float32:
            reject("requires_float32_input", field, "mixed residual stream requires FP32 input")
        elif not supported_width(context.d_model, torch.float32):
            reject("unsupported_shape", field, "HIP mixed norm has no kernel for this width")
        if (
            config.program.attention_output_projection not in _FP16_PROJECTIONS
            or config.program.ffn_output_projection not in _FP16_PROJECTIONS
        ):
            reject(
                "requires_fp16_update",
                "program.precision_plan",
                "mixed residual norm requires FP16 attention and FFN updates",
            )

    @staticmethod
    def _validate_linear_boundary(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        """The fused Linear + residual + LayerNorm boundary at both residual
        boundaries of a layer (the reference's TRITON_LINEAR_MIXED rules,
        solution/plan_builder.py:668-707, 796-801, 950-990), on a 16-bit
        stream with native-dtype output projections."""

        from .kernels.boundary.hip_linear_residual_norm import launch_config_is_valid, supported_width

        field = "program.residual_norm"
        _validate_hip_common(context, hardware, hardware.hip_linear_residual_norm, field, reject)
        if context.dtype not in {torch.float16, torch.bfloat16}:
            reject("unsupported_dtype", field, "the HIP linear boundary runs on FP16 and BF16 streams")
        for name in ("attention_output_projection", "ffn_output_projection"):
            if getattr(config.program, name) is not ProjectionBackend.INPUT_DTYPE:
                reject(
                    "backend_incompatible",
                    f"program.{name}",
                    "the HIP linear boundary multiplies the native-dtype projection weights",
                )
        if not supported_width(context.d_model, context.d_model) or (
            context.ffn_dim is None or not supported_width(context.d_model, context.ffn_dim)
        ):
            reject(
                "unsupported_shape",
                field,
                "the HIP linear boundary supports d_model 512 and 1024 with ffn_dim % 64 == 0",
            )
        if config.schedule.runtime is RuntimeBackend.COMPILED_FORWARD:
            reject("runtime_incompatible", "schedule.runtime", "the linear boundary is not nested in compiled forward")
        launch = config.schedule.residual_norm_launch
        assert launch is not None
        if not launch_config_is_valid(context.d_model, launch.block_rows, launch.num_warps):
            reject(
                "unsupported_launch_value",
                "schedule.residual_norm_launch",
                "the HIP linear boundary runs 65536 / d_model rows per workgroup of 8 wavefronts",
            )

    # ------------------------------------------------------------- initial norm
    @staticmethod
    def _validate_initial_norm(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        backend = config.program.initial_norm
        if backend is InitialNormBackend.TORCH:
            return
        if backend is InitialNormBackend.HIP_FUSED_QKV:
            PlanBuilder._validate_fused_initial_norm_qkv(config, context, hardware, reject)
            return
        if backend is not InitialNormBackend.HIP:
            _unavailable(reject, "program.initial_norm", f"Triton initial norm {backend.value}")
            return
        from .kernels.norm.hip_residual import launch_config_is_valid, supported_width

        field = "program.initial_norm"
        _validate_hip_common(context, hardware, hardware.hip_initial_norm, field, reject)
        launch = config.schedule.initial_norm_launch
        assert launch is not None
        if not launch_config_is_valid(launch.block_rows, launch.num_warps):
            reject(
                "unsupported_launch_value",
                "schedule.initial_norm_launch",
                "HIP norm needs block_rows a multiple of num_warps and at most 64",
            )
        if context.dtype not in {torch.float32, torch.float16, torch.bfloat16}:
            reject("unsupported_dtype", field, "HIP initial norm supports FP32, FP16 and BF16 inputs")
        elif not supported_width(context.d_model, context.dtype):
            reject("unsupported_shape", field, "HIP initial norm has no kernel for this width")

    @staticmethod
    def _validate_fused_initial_norm_qkv(
        config: ConfigSpec,
        context: ExecutionContext,
        hardware: HardwareCapabilities,
        reject: Reject,
    ) -> None:
        """The reference's TRITON_FUSED_QKV rules (solution/plan_builder.py:
        1100-1159) for the gfx950 kernel: no launch of its own, the
        native-layout QKV projection, no mask; its own shape domain (16-bit
        models of width 512-4096) instead of the reference's one fp32 shape,
        and any runtime."""

        from .kernels.projection.hip_qkv_layout import INITIAL_NORM_WIDTHS

        field = "program.initial_norm"
        if config.schedule.initial_norm_launch is not None:
            reject(
                "launch_incompatible",
                "schedule.initial_norm_launch",
                "the fused initial norm uses the QKV launch configuration",
            )
        _validate_hip_common(context, hardware, hardware.hip_qkv_native_bhsd, field, reject)
        if config.program.qkv_materialization is not QKVMaterialization.HIP_NATIVE_BHSD:
            reject(
                "qkv_incompatible",
                field,
                "the fused initial norm requires the HIP native-layout QKV projection",
            )
        if context.dtype not in {torch.float16, torch.bfloat16}:
            reject("unsupported_dtype", field, "the fused initial norm runs on FP16 and BF16 models")
        if context.d_model not in INITIAL_NORM_WIDTHS:
            reject(
                "unsupported_shape",
                field,
                "the fused initial norm supports d_model 512, 1024, 2048 and 4096",
            )

    # -------------------------------------------------------------------- build
    @staticmethod
    def _build_plan(
        config: ConfigSpec,
        outer: ExecutionContext,
        inner: ExecutionContext,
        hardware: HardwareCapabilities,
    ) -> ExecutionPlan:
        program, schedule = config.program, config.schedule
        qkv_dtype = PlanBuilder._projection_dtype(program.qkv_projection, inner)
        out_dtype = PlanBuilder._projection_dtype(program.attention_output_projection, inner)
        ffn_in_dtype = PlanBuilder._projection_dtype(program.ffn_input_projection, inner)
        ffn_out_dtype = PlanBuilder._projection_dtype(program.ffn_output_projection, inner)
        if program.precision_plan in {
            PrecisionPlan.FP16_FFN_INPUT_FP32_GELU,
            PrecisionPlan.FP16_ATTENTION_AND_FFN_INPUT,
        }:
            activation_dtype = "float32"
        else:
            activation_dtype = ffn_in_dtype
        if program.attention in TRITON_ATTENTION_BACKENDS or program.attention in {
            AttentionBackend.FP16_EFFICIENT_SDPA,
            AttentionBackend.FP16_CUDNN_SDPA,
        }:
            attention_dtype = "float16"
        else:
            attention_dtype = qkv_dtype
        layers = max(0, int(inner.num_layers or 0))
        expected = ExpectedExecutionTrace(
            runtime_backend=schedule.runtime,
            attention_backend=program.attention,
            qkv_projection_backend=program.qkv_projection,
            attention_output_projection_backend=program.attention_output_projection,
            ffn_input_projection_backend=program.ffn_input_projection,
            ffn_output_projection_backend=program.ffn_output_projection,
            precision_plan=program.precision_plan,
            qkv_materialization=program.qkv_materialization,
            attention_output_bridge=program.attention_output_bridge,
            attention_output_layout=config.attention_output_layout,
            ffn_backend=program.ffn,
            residual_norm_backend=program.residual_norm,
            initial_norm_backend=program.initial_norm,
            attention_compute_dtype=attention_dtype,
            qkv_projection_compute_dtype=qkv_dtype,
            attention_output_projection_compute_dtype=out_dtype,
            ffn_input_projection_compute_dtype=ffn_in_dtype,
            ffn_activation_output_dtype=activation_dtype,
            ffn_output_projection_compute_dtype=ffn_out_dtype,
            attention_calls=layers,
            qkv_projection_calls=layers,
            qkv_materialization_calls=layers,
            attention_output_bridge_calls=layers,
            attention_output_projection_calls=layers,
            ffn_calls=layers,
            ffn_input_projection_calls=layers,
            ffn_output_projection_calls=layers,
            residual_norm_calls=2 * layers,
            initial_norm_calls=1 if layers else 0,
            runtime_calls=1,
            attention_launch=schedule.attention_launch,
            qkv_launch=schedule.qkv_launch,
            attention_output_projection_launch=schedule.attention_output_projection_launch,
            residual_norm_launch=schedule.residual_norm_launch,
            initial_norm_launch=schedule.initial_norm_launch,
            ffn_launch=schedule.ffn_launch,
            ffn_input_launch=schedule.ffn_input_launch,
        )
        return ExecutionPlan(
            config=config,
            outer_context=outer,
            inner_context=inner,
            attention_backend=program.attention,
            attention_compute_dtype=attention_dtype,
            qkv_projection_backend=program.qkv_projection,
            qkv_projection_compute_dtype=qkv_dtype,
            qkv_materialization=program.qkv_materialization,
            attention_output_bridge=program.attention_output_bridge,
            attention_output_layout=config.attention_output_layout,
            attention_output_projection_backend=program.attention_output_projection,
            attention_output_projection_compute_dtype=out_dtype,
            ffn_backend=program.ffn,
            ffn_input_projection_backend=program.ffn_input_projection,
            ffn_input_projection_compute_dtype=ffn_in_dtype,
            ffn_activation_output_dtype=activation_dtype,
            ffn_output_projection_backend=program.ffn_output_projection,
            ffn_output_projection_compute_dtype=ffn_out_dtype,
            precision_plan=program.precision_plan,
            residual_norm_backend=program.residual_norm,
            initial_norm_backend=program.initial_norm,
            runtime_backend=schedule.runtime,
            compile_mode=schedule.compile_mode,
            batch_tile_size=schedule.batch_tile_size,
            microbatch_size=schedule.microbatch_size,
            reuse_unchanged_input=schedule.reuse_unchanged_input,
            attention_launch=schedule.attention_launch,
            qkv_launch=schedule.qkv_launch,
            attention_output_projection_launch=schedule.attention_output_projection_launch,
            residual_norm_launch=schedule.residual_norm_launch,
            initial_norm_launch=schedule.initial_norm_launch,
            ffn_launch=schedule.ffn_launch,
            ffn_input_launch=schedule.ffn_input_launch,
            use_d32_residual_norm=False,
            use_masked_residual_norm=False,
            use_masked_initial_norm=False,
            expected_trace=expected,
        )

    @staticmethod
    def _projection_dtype(backend: ProjectionBackend, context: ExecutionContext) -> str:
        if backend in _FP16_PROJECTIONS:
            return "float16"
        return context.dtype_name


def _validate_hip_common(
    context: ExecutionContext,
    hardware: HardwareCapabilities,
    capability: bool | None,
    field: str,
    reject: Reject,
) -> None:
    if not capability:
        reject("backend_unavailable", field, "the gfx950 HIP library is not loaded")
    if context.device.type != "cuda" or not hardware.is_gfx950:
        reject("requires_gfx950", field, "HIP kernels require an MI355X (gfx950) GPU")
    if not context.inference:
        reject("requires_inference", field, "HIP kernels are available only for inference")
    if context.has_valid_token_mask:
        reject("mask_not_supported", field, "HIP norms run on all-valid workloads")


__all__ = [
    "CompilationResult",
    "CompileRejection",
    "ConfigRejectedError",
    "ConstraintViolation",
    "HardwareCapabilities",
    "PlanBuilder",
]
