"""Typed, serializable execution programs for the Transformer forward.

Keeps the reference's plan format (solution/config.py:1-846) so that configs
written by either side parse on the other and keep their ``config_id``:
the same enums and string values, the same exact-field JSON objects, the same
canonical JSON (sorted keys, compact separators, ASCII, no NaN) hashed with
SHA-256 into ``cfg-<hex>`` (reference :753-785), and the same cross-field
presence rules (reference :692-740).

Additions for the gfx950 backends, all of which reuse existing JSON fields so
the schema (version 4) is unchanged:

* ``AttentionBackend.HIP_STREAMING_DH64`` - hand-written MFMA causal attention
  (head_dim 64, bf16/fp16, direct BSD output); its launch parameters live in
  ``attention_launch`` (block_m query rows per workgroup, block_n keys per
  tile, num_warps wave64 wavefronts per workgroup, num_stages LDS buffers).
* ``ResidualNormBackend.HIP_FUSED`` (same-dtype residual stream) and
  ``ResidualNormBackend.HIP_MIXED`` (fp32 stream, 16-bit update) - the fused
  residual + LayerNorm kernel; launch in ``residual_norm_launch`` (block_rows
  rows per workgroup of num_warps wavefronts).
* ``InitialNormBackend.HIP`` - the layer-0 LayerNorm; launch in
  ``initial_norm_launch``.
* ``FFNBackend.HIP_FUSED_MLP_BOUNDARY`` - the whole FFN fused through its
  residual add and LayerNorm (the reference's ``TRITON_FUSED_MLP_BOUNDARY``);
  like it, the kernel's launch is ``residual_norm_launch``.
* ``InitialNormBackend.HIP_FUSED_QKV`` - the layer-0 LayerNorm fused into the
  HIP native-layout QKV projection (the reference's ``TRITON_FUSED_QKV``);
  like it, no ``initial_norm_launch``: it runs with ``qkv_launch``.

Python 3.10 has no ``enum.StrEnum``; ``str``-mixin enums serialize through
``.value`` exactly like the reference's StrEnum members.
"""

from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from enum import Enum
from typing import Any, ClassVar

CONFIG_SCHEMA_VERSION = 4


class _StrEnum(str, Enum):
    def __str__(self) -> str:
        return str(self.value)


class AttentionBackend(_StrEnum):
    """Implemented attention primitives."""

    REFERENCE_STREAMING = "reference_streaming"
    CAUSAL_SDPA = "causal_sdpa"
    FP16_EFFICIENT_SDPA = "fp16_efficient_sdpa"
    FP16_CUDNN_SDPA = "fp16_cudnn_sdpa"
    TRITON_SHAPE13 = "triton_shape13"
    TRITON_DH8 = "triton_dh8"
    TRITON_STREAMING_DH64 = "triton_streaming_dh64"
    HIP_STREAMING_DH64 = "hip_streaming_dh64"


class ProjectionBackend(_StrEnum):
    """Per-role projection execution and weight-storage choices."""

    INPUT_DTYPE = "input_dtype"
    AUTOCAST_FP16 = "autocast_fp16"
    FP16_SHADOW = "fp16_shadow"


class PrecisionPlan(_StrEnum):
    """Finite projection/cast graphs."""

    INPUT_DTYPE = "input_dtype"
    FP16_QKV_ATTENTION = "fp16_qkv_attention"
    FP16_ATTENTION_BRANCH = "fp16_attention_branch"
    FP16_FFN_INPUT_FP32_GELU = "fp16_ffn_input_fp32_gelu"
    FP16_ATTENTION_AND_FFN_INPUT = "fp16_attention_and_ffn_input"
    FP16_FFN_BRANCH = "fp16_ffn_branch"
    FP16_FFN_OUTPUT = "fp16_ffn_output"
    FP16_CORE = "fp16_core"


class QKVMaterialization(_StrEnum):
    VIEW = "view"
    CONTIGUOUS = "contiguous"
    TRITON_NATIVE_BHSD = "triton_native_bhsd"
    HIP_NATIVE_BHSD = "hip_native_bhsd"


class AttentionOutputBridge(_StrEnum):
    TORCH_BHSD_TO_BSD = "torch_bhsd_to_bsd"
    ATTENTION_DIRECT_BSD = "attention_direct_bsd"
    TRITON_BHSD_PROJECTION = "triton_bhsd_projection"


class FFNBackend(_StrEnum):
    TORCH = "torch"
    COMPILED = "compiled"
    TRITON_EXACT_GELU = "triton_exact_gelu"
    TRITON_LINEAR_EXACT_GELU = "triton_linear_exact_gelu"
    TRITON_FUSED_MLP_BOUNDARY = "triton_fused_mlp_boundary"
    HIP_LINEAR_EXACT_GELU = "hip_linear_exact_gelu"
    HIP_EXACT_GELU = "hip_exact_gelu"
    HIP_FUSED_MLP_BOUNDARY = "hip_fused_mlp_boundary"


class ResidualNormBackend(_StrEnum):
    TORCH = "torch"
    COMPILED = "compiled"
    TRITON = "triton"
    TRITON_MIXED = "triton_mixed"
    TRITON_LINEAR_MIXED = "triton_linear_mixed"
    HIP_FUSED = "hip_fused"
    HIP_MIXED = "hip_mixed"
    HIP_LINEAR_FUSED = "hip_linear_fused"


class InitialNormBackend(_StrEnum):
    TORCH = "torch"
    TRITON_FP16 = "triton_fp16"
    TRITON_FUSED_QKV = "triton_fused_qkv"
    HIP = "hip"
    HIP_FUSED_QKV = "hip_fused_qkv"


class RuntimeBackend(_StrEnum):
    EAGER = "eager"
    CUDA_GRAPH = "cuda_graph"
    BATCH_TILED_CUDA_GRAPH = "batch_tiled_cuda_graph"
    COMPILED_FORWARD = "compiled_forward"
    STREAMED = "streamed"


class AttentionOutputLayout(_StrEnum):
    BHSD = "bhsd"
    BSD = "bsd"


TRITON_ATTENTION_BACKENDS = frozenset(
    {
        AttentionBackend.TRITON_SHAPE13,
        AttentionBackend.TRITON_DH8,
        AttentionBackend.TRITON_STREAMING_DH64,
    }
)
HIP_ATTENTION_BACKENDS = frozenset({AttentionBackend.HIP_STREAMING_DH64})
# Backends whose kernels run an online causal softmax and need attention_launch.
LAUNCHED_ATTENTION_BACKENDS = TRITON_ATTENTION_BACKENDS | HIP_ATTENTION_BACKENDS
# Backends that write [B, S, H*Dh] directly.
DIRECT_BSD_ATTENTION_BACKENDS = LAUNCHED_ATTENTION_BACKENDS
HIP_RESIDUAL_NORM_BACKENDS = frozenset(
    {
        ResidualNormBackend.HIP_FUSED,
        ResidualNormBackend.HIP_MIXED,
        ResidualNormBackend.HIP_LINEAR_FUSED,
    }
)
# Backends that fuse the branch's output projection into the residual
# boundary (the update never reaches HBM).
LINEAR_BOUNDARY_RESIDUAL_NORM_BACKENDS = frozenset(
    {ResidualNormBackend.TRITON_LINEAR_MIXED, ResidualNormBackend.HIP_LINEAR_FUSED}
)
LAUNCHED_RESIDUAL_NORM_BACKENDS = frozenset(
    {
        ResidualNormBackend.TRITON,
        ResidualNormBackend.TRITON_MIXED,
        ResidualNormBackend.TRITON_LINEAR_MIXED,
    }
) | HIP_RESIDUAL_NORM_BACKENDS
LAUNCHED_INITIAL_NORM_BACKENDS = frozenset(
    {InitialNormBackend.TRITON_FP16, InitialNormBackend.HIP}
)
# QKV materializations produced by a projection kernel (they need qkv_launch).
NATIVE_QKV_MATERIALIZATIONS = frozenset(
    {QKVMaterialization.TRITON_NATIVE_BHSD, QKVMaterialization.HIP_NATIVE_BHSD}
)

_PROJECTION_FIELDS = (
    "qkv_projection",
    "attention_output_projection",
    "ffn_input_projection",
    "ffn_output_projection",
)

_PRECISION_FP16_PROJECTIONS = {
    PrecisionPlan.INPUT_DTYPE: frozenset(),
    PrecisionPlan.FP16_QKV_ATTENTION: frozenset({"qkv_projection"}),
    PrecisionPlan.FP16_ATTENTION_BRANCH: frozenset(
        {"qkv_projection", "attention_output_projection"}
    ),
    PrecisionPlan.FP16_FFN_INPUT_FP32_GELU: frozenset({"ffn_input_projection"}),
    PrecisionPlan.FP16_ATTENTION_AND_FFN_INPUT: frozenset(
        {"qkv_projection", "attention_output_projection", "ffn_input_projection"}
    ),
    PrecisionPlan.FP16_FFN_BRANCH: frozenset(
        {"ffn_input_projection", "ffn_output_projection"}
    ),
    PrecisionPlan.FP16_FFN_OUTPUT: frozenset({"ffn_output_projection"}),
    PrecisionPlan.FP16_CORE: frozenset(_PROJECTION_FIELDS),
}


def fp16_projection_fields(precision_plan: PrecisionPlan) -> frozenset[str]:
    """Projection roles executed in FP16 under one precision graph."""

    return _PRECISION_FP16_PROJECTIONS[PrecisionPlan(precision_plan)]


COMPILED_FORWARD_MODES = frozenset(
    {"max-autotune", "max-autotune-no-cudagraphs", "reduce-overhead"}
)
DEFAULT_COMPILED_FORWARD_MODE = "max-autotune"


# ---------------------------------------------------------------------------
# field validation helpers


def _positive_int(value: object, *, field: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"{field} must be a positive integer")
    return value


def _power_of_two(value: object, *, field: str) -> int:
    number = _positive_int(value, field=field)
    if number & (number - 1):
        raise ValueError(f"{field} must be a power of two")
    return number


def _stage_count(value: object, *, field: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or not 1 <= value <= 8:
        raise ValueError(f"{field} must be in [1, 8]")
    return value


def _warp_count(value: object, *, field: str) -> int:
    if isinstance(value, bool) or value not in {1, 2, 4, 8}:
        raise ValueError(f"{field} must be one of 1, 2, 4, 8")
    return int(value)  # type: ignore[arg-type]


def _mapping(value: object, *, field: str) -> dict[str, Any]:
    if not isinstance(value, dict):
        raise TypeError(f"{field} must be an object")
    return value


def _exact_fields(value: dict[str, Any], expected: frozenset[str], *, field: str) -> None:
    missing = expected - set(value)
    unknown = set(value) - expected
    if missing or unknown:
        raise ValueError(
            f"invalid {field} fields; missing={sorted(missing)}; unknown={sorted(unknown)}"
        )


class _LaunchParams:
    """Shared to_dict/from_dict for the flat integer launch objects."""

    _FIELD_ORDER: ClassVar[tuple[str, ...]] = ()
    _JSON_NAME: ClassVar[str] = ""

    def to_dict(self) -> dict[str, int]:
        return {name: getattr(self, name) for name in self._FIELD_ORDER}

    @classmethod
    def from_dict(cls, payload: object):  # type: ignore[no-untyped-def]
        value = _mapping(payload, field=cls._JSON_NAME)
        _exact_fields(value, frozenset(cls._FIELD_ORDER), field=cls._JSON_NAME)
        return cls(**value)


@dataclass(frozen=True, slots=True)
class AttentionLaunchParams(_LaunchParams):
    """Launch of a tiled attention kernel (reference TritonAttentionParams,
    solution/config.py:189-234).  For the HIP kernel num_warps counts wave64
    wavefronts and num_stages LDS tile buffers."""

    block_m: int
    block_n: int
    num_warps: int
    num_stages: int

    _FIELD_ORDER: ClassVar[tuple[str, ...]] = ("block_m", "block_n", "num_warps", "num_stages")
    _JSON_NAME: ClassVar[str] = "attention_launch"

    def __post_init__(self) -> None:
        object.__setattr__(self, "block_m", _power_of_two(self.block_m, field="attention_launch.block_m"))
        object.__setattr__(self, "block_n", _power_of_two(self.block_n, field="attention_launch.block_n"))
        _warp_count(self.num_warps, field="attention_launch.num_warps")
        _stage_count(self.num_stages, field="attention_launch.num_stages")


@dataclass(frozen=True, slots=True)
class QKVLaunchParams(_LaunchParams):
    """Reference TritonQKVParams (solution/config.py:237-271)."""

    block_m: int
    block_n: int
    block_k: int
    num_warps: int

    _FIELD_ORDER: ClassVar[tuple[str, ...]] = ("block_m", "block_n", "block_k", "num_warps")
    _JSON_NAME: ClassVar[str] = "qkv_launch"

    def __post_init__(self) -> None:
        for name in ("block_m", "block_n", "block_k"):
            object.__setattr__(self, name, _power_of_two(getattr(self, name), field=f"qkv_launch.{name}"))
        _warp_count(self.num_warps, field="qkv_launch.num_warps")


@dataclass(frozen=True, slots=True)
class GemmLaunchParams(_LaunchParams):
    """Reference TritonGemmParams (solution/config.py:274-324)."""

    block_m: int
    block_n: int
    block_k: int
    num_warps: int
    num_stages: int

    _FIELD_ORDER: ClassVar[tuple[str, ...]] = (
        "block_m", "block_n", "block_k", "num_warps", "num_stages",
    )
    _JSON_NAME: ClassVar[str] = "gemm_launch"

    def __post_init__(self) -> None:
        for name in ("block_m", "block_n", "block_k"):
            object.__setattr__(self, name, _power_of_two(getattr(self, name), field=f"gemm_launch.{name}"))
        _warp_count(self.num_warps, field="gemm_launch.num_warps")
        _stage_count(self.num_stages, field="gemm_launch.num_stages")


@dataclass(frozen=True, slots=True)
class NormLaunchParams(_LaunchParams):
    """Launch of a row-blocked norm kernel (reference TritonNormParams,
    solution/config.py:327-355): block_rows rows per workgroup of num_warps
    wavefronts."""

    block_rows: int
    num_warps: int

    _FIELD_ORDER: ClassVar[tuple[str, ...]] = ("block_rows", "num_warps")
    _JSON_NAME: ClassVar[str] = "norm_launch"

    def __post_init__(self) -> None:
        object.__setattr__(self, "block_rows", _power_of_two(self.block_rows, field="norm_launch.block_rows"))
        _warp_count(self.num_warps, field="norm_launch.num_warps")


@dataclass(frozen=True, slots=True)
class FFNLaunchParams(_LaunchParams):
    """Reference TritonFFNParams (solution/config.py:358-386)."""

    block_size: int
    num_warps: int

    _FIELD_ORDER: ClassVar[tuple[str, ...]] = ("block_size", "num_warps")
    _JSON_NAME: ClassVar[str] = "ffn_launch"

    def __post_init__(self) -> None:
        object.__setattr__(self, "block_size", _power_of_two(self.block_size, field="ffn_launch.block_size"))
        _warp_count(self.num_warps, field="ffn_launch.num_warps")


# The reference's names for the same launch objects (drop-in imports).
TritonAttentionParams = AttentionLaunchParams
TritonQKVParams = QKVLaunchParams
TritonGemmParams = GemmLaunchParams
TritonNormParams = NormLaunchParams
TritonFFNParams = FFNLaunchParams


@dataclass(frozen=True, slots=True)
class ProgramConfig:
    """High-level execution structure (reference solution/config.py:389-487)."""

    attention: AttentionBackend
    qkv_projection: ProjectionBackend
    attention_output_projection: ProjectionBackend
    ffn_input_projection: ProjectionBackend
    ffn_output_projection: ProjectionBackend
    precision_plan: PrecisionPlan
    qkv_materialization: QKVMaterialization
    attention_output_bridge: AttentionOutputBridge
    ffn: FFNBackend
    residual_norm: ResidualNormBackend
    initial_norm: InitialNormBackend = InitialNormBackend.TORCH

    _FIELD_TYPES: ClassVar[dict[str, type]] = {
        "attention": AttentionBackend,
        "qkv_projection": ProjectionBackend,
        "attention_output_projection": ProjectionBackend,
        "ffn_input_projection": ProjectionBackend,
        "ffn_output_projection": ProjectionBackend,
        "precision_plan": PrecisionPlan,
        "qkv_materialization": QKVMaterialization,
        "attention_output_bridge": AttentionOutputBridge,
        "ffn": FFNBackend,
        "residual_norm": ResidualNormBackend,
        "initial_norm": InitialNormBackend,
    }

    def __post_init__(self) -> None:
        for name, enum_type in self._FIELD_TYPES.items():
            object.__setattr__(self, name, enum_type(getattr(self, name)))
        fp16_fields = _PRECISION_FP16_PROJECTIONS[self.precision_plan]
        fp16_backends = {ProjectionBackend.AUTOCAST_FP16, ProjectionBackend.FP16_SHADOW}
        for name in _PROJECTION_FIELDS:
            backend = getattr(self, name)
            if name in fp16_fields:
                if backend not in fp16_backends:
                    raise ValueError(
                        f"{name} must use an FP16 backend for "
                        f"precision_plan={self.precision_plan.value}"
                    )
            elif backend is not ProjectionBackend.INPUT_DTYPE:
                raise ValueError(
                    f"{name} must use input_dtype for precision_plan={self.precision_plan.value}"
                )

    def to_dict(self) -> dict[str, str]:
        return {name: getattr(self, name).value for name in self._FIELD_TYPES}

    @classmethod
    def from_dict(cls, payload: object) -> ProgramConfig:
        value = _mapping(payload, field="program")
        _exact_fields(value, frozenset(cls._FIELD_TYPES), field="program")
        return cls(**value)


_SCHEDULE_LAUNCH_TYPES: dict[str, type] = {
    "attention_launch": AttentionLaunchParams,
    "qkv_launch": QKVLaunchParams,
    "attention_output_projection_launch": GemmLaunchParams,
    "residual_norm_launch": NormLaunchParams,
    "initial_norm_launch": NormLaunchParams,
    "ffn_launch": FFNLaunchParams,
    "ffn_input_launch": GemmLaunchParams,
}


@dataclass(frozen=True, slots=True)
class ScheduleConfig:
    """Runtime and conditional launch parameters (reference :490-669)."""

    runtime: RuntimeBackend
    attention_launch: AttentionLaunchParams | None = None
    qkv_launch: QKVLaunchParams | None = None
    attention_output_projection_launch: GemmLaunchParams | None = None
    residual_norm_launch: NormLaunchParams | None = None
    initial_norm_launch: NormLaunchParams | None = None
    ffn_launch: FFNLaunchParams | None = None
    ffn_input_launch: GemmLaunchParams | None = None
    compile_mode: str | None = None
    batch_tile_size: int | None = None
    microbatch_size: int | None = None
    reuse_unchanged_input: bool = False

    _FIELDS: ClassVar[tuple[str, ...]] = (
        "runtime",
        *_SCHEDULE_LAUNCH_TYPES,
        "compile_mode",
        "batch_tile_size",
        "microbatch_size",
        "reuse_unchanged_input",
    )

    def __post_init__(self) -> None:
        runtime = RuntimeBackend(self.runtime)
        object.__setattr__(self, "runtime", runtime)
        for name, launch_type in _SCHEDULE_LAUNCH_TYPES.items():
            value = getattr(self, name)
            if value is not None and not isinstance(value, launch_type):
                raise TypeError(f"{name} must be {launch_type.__name__} or None")
        mode = self.compile_mode
        if runtime is RuntimeBackend.COMPILED_FORWARD:
            if mode is None:
                mode = DEFAULT_COMPILED_FORWARD_MODE
                object.__setattr__(self, "compile_mode", mode)
            if mode not in COMPILED_FORWARD_MODES:
                raise ValueError(f"unsupported compile_mode: {mode}")
        elif mode is not None:
            raise ValueError("compile_mode is valid only for compiled_forward")
        if runtime is RuntimeBackend.BATCH_TILED_CUDA_GRAPH:
            object.__setattr__(
                self, "batch_tile_size", _positive_int(self.batch_tile_size, field="batch_tile_size")
            )
        elif self.batch_tile_size is not None:
            raise ValueError("batch_tile_size is valid only for batch_tiled_cuda_graph")
        if runtime is RuntimeBackend.STREAMED:
            object.__setattr__(
                self, "microbatch_size", _positive_int(self.microbatch_size, field="microbatch_size")
            )
        elif self.microbatch_size is not None:
            raise ValueError("microbatch_size is valid only for the streamed runtime")
        if not isinstance(self.reuse_unchanged_input, bool):
            raise TypeError("reuse_unchanged_input must be a bool")
        if self.reuse_unchanged_input and runtime is not RuntimeBackend.CUDA_GRAPH:
            raise ValueError("reuse_unchanged_input is valid only for the cuda_graph runtime")

    def to_dict(self) -> dict[str, Any]:
        payload: dict[str, Any] = {"runtime": self.runtime.value}
        for name in _SCHEDULE_LAUNCH_TYPES:
            value = getattr(self, name)
            payload[name] = None if value is None else value.to_dict()
        payload["compile_mode"] = self.compile_mode
        payload["batch_tile_size"] = self.batch_tile_size
        payload["microbatch_size"] = self.microbatch_size
        payload["reuse_unchanged_input"] = self.reuse_unchanged_input
        return payload

    @classmethod
    def from_dict(cls, payload: object) -> ScheduleConfig:
        value = _mapping(payload, field="schedule")
        _exact_fields(value, frozenset(cls._FIELDS), field="schedule")
        launches = {
            name: None if value[name] is None else launch_type.from_dict(value[name])
            for name, launch_type in _SCHEDULE_LAUNCH_TYPES.items()
        }
        return cls(
            runtime=value["runtime"],
            **launches,
            compile_mode=value["compile_mode"],
            batch_tile_size=value["batch_tile_size"],
            microbatch_size=value["microbatch_size"],
            reuse_unchanged_input=value["reuse_unchanged_input"],
        )


@dataclass(frozen=True, slots=True)
class ConfigSpec:
    """Canonical program plus schedule (reference solution/config.py:672-785)."""

    program: ProgramConfig
    schedule: ScheduleConfig
    schema_version: int = CONFIG_SCHEMA_VERSION

    _FIELDS: ClassVar[frozenset[str]] = frozenset({"schema_version", "program", "schedule"})

    def __post_init__(self) -> None:
        if self.schema_version != CONFIG_SCHEMA_VERSION:
            raise ValueError(f"schema_version must be {CONFIG_SCHEMA_VERSION}")
        if not isinstance(self.program, ProgramConfig):
            raise TypeError("program must be ProgramConfig")
        if not isinstance(self.schedule, ScheduleConfig):
            raise TypeError("schedule must be ScheduleConfig")
        program, schedule = self.program, self.schedule

        launched_attention = program.attention in LAUNCHED_ATTENTION_BACKENDS
        if launched_attention != (schedule.attention_launch is not None):
            raise ValueError(
                "attention_launch must be present exactly for Triton or HIP attention"
            )
        native_qkv = program.qkv_materialization in NATIVE_QKV_MATERIALIZATIONS
        if native_qkv != (schedule.qkv_launch is not None):
            raise ValueError("qkv_launch must be present exactly for Triton or HIP native QKV")
        fused_output_projection = (
            program.attention_output_bridge is AttentionOutputBridge.TRITON_BHSD_PROJECTION
            and program.residual_norm is not ResidualNormBackend.TRITON_LINEAR_MIXED
        )
        if fused_output_projection != (schedule.attention_output_projection_launch is not None):
            raise ValueError(
                "attention_output_projection_launch must be present exactly for "
                "the Triton BHSD projection bridge"
            )
        launched_residual = program.residual_norm in LAUNCHED_RESIDUAL_NORM_BACKENDS
        if launched_residual != (schedule.residual_norm_launch is not None):
            raise ValueError(
                "residual_norm_launch must be present exactly for Triton or HIP residual norm"
            )
        launched_initial = program.initial_norm in LAUNCHED_INITIAL_NORM_BACKENDS
        if launched_initial != (schedule.initial_norm_launch is not None):
            raise ValueError(
                "initial_norm_launch must be present exactly for Triton or HIP initial norm"
            )
        elementwise_gelu = program.ffn in {FFNBackend.TRITON_EXACT_GELU, FFNBackend.HIP_EXACT_GELU}
        if elementwise_gelu != (schedule.ffn_launch is not None):
            raise ValueError("ffn_launch must be present exactly for Triton or HIP Exact-GELU")
        fused_ffn_input = program.ffn in {
            FFNBackend.TRITON_LINEAR_EXACT_GELU,
            FFNBackend.HIP_LINEAR_EXACT_GELU,
        }
        if fused_ffn_input != (schedule.ffn_input_launch is not None):
            raise ValueError(
                "ffn_input_launch must be present exactly for Triton or HIP Linear Exact-GELU"
            )

    @property
    def attention_output_layout(self) -> AttentionOutputLayout:
        if self.program.attention_output_bridge is AttentionOutputBridge.ATTENTION_DIRECT_BSD:
            return AttentionOutputLayout.BSD
        return AttentionOutputLayout.BHSD

    def to_dict(self) -> dict[str, Any]:
        return {
            "schema_version": self.schema_version,
            "program": self.program.to_dict(),
            "schedule": self.schedule.to_dict(),
        }

    def canonical_json(self) -> str:
        return json.dumps(
            self.to_dict(),
            ensure_ascii=True,
            allow_nan=False,
            sort_keys=True,
            separators=(",", ":"),
        )

    @property
    def sha256(self) -> str:
        return hashlib.sha256(self.canonical_json().encode("utf-8")).hexdigest()

    @property
    def config_id(self) -> str:
        return f"cfg-{self.sha256}"

    @classmethod
    def from_dict(cls, payload: object) -> ConfigSpec:
        value = _mapping(payload, field="config")
        _exact_fields(value, cls._FIELDS, field="config")
        return cls(
            schema_version=value["schema_version"],
            program=ProgramConfig.from_dict(value["program"]),
            schedule=ScheduleConfig.from_dict(value["schedule"]),
        )


def portable_config() -> ConfigSpec:
    """The explicit reference-order program (reference :788-806)."""

    return ConfigSpec(
        program=ProgramConfig(
            attention=AttentionBackend.REFERENCE_STREAMING,
            qkv_projection=ProjectionBackend.INPUT_DTYPE,
            attention_output_projection=ProjectionBackend.INPUT_DTYPE,
            ffn_input_projection=ProjectionBackend.INPUT_DTYPE,
            ffn_output_projection=ProjectionBackend.INPUT_DTYPE,
            precision_plan=PrecisionPlan.INPUT_DTYPE,
            qkv_materialization=QKVMaterialization.VIEW,
            attention_output_bridge=AttentionOutputBridge.TORCH_BHSD_TO_BSD,
            ffn=FFNBackend.TORCH,
            residual_norm=ResidualNormBackend.TORCH,
            initial_norm=InitialNormBackend.TORCH,
        ),
        schedule=ScheduleConfig(runtime=RuntimeBackend.EAGER),
    )


def portable_streamed_config(*, microbatch_size: int = 1) -> ConfigSpec:
    """The reference program under the streamed schedule (reference :809-818)."""

    return ConfigSpec(
        program=portable_config().program,
        schedule=ScheduleConfig(runtime=RuntimeBackend.STREAMED, microbatch_size=microbatch_size),
    )


HIP_DEFAULT_ATTENTION_LAUNCH = AttentionLaunchParams(
    block_m=128, block_n=64, num_warps=4, num_stages=2
)
# Long sequences: 256-row query tiles shared by 8 wavefronts, which halves the
# K/V tile loads, LDS stores and barriers per FLOP against 128-row tiles
# (measured fastest of the 4/8-wave, 32/64-rows-per-wave launches on the
# 100k-token chunk).  Short sequences keep 128-row tiles, which give twice as
# many workgroups to fill 256 CUs.
HIP_LONG_SEQUENCE_ATTENTION_LAUNCH = AttentionLaunchParams(
    block_m=256, block_n=64, num_warps=8, num_stages=2
)
HIP_DEFAULT_NORM_LAUNCH = NormLaunchParams(block_rows=4, num_warps=4)


# The launch of the HIP Linear + exact-GELU kernel (csrc/linear_gelu.hip).
HIP_LINEAR_LAUNCH = GemmLaunchParams(block_m=256, block_n=256, block_k=64, num_warps=8, num_stages=2)
# The default launch of the HIP elementwise exact GELU (csrc/gelu.hip): one
# 16-byte chunk per thread, 8 wavefronts (6.1 TB/s on the C5 hidden tensor,
# the fastest of the implemented launches on MI355X).
HIP_GELU_LAUNCH = FFNLaunchParams(block_size=4096, num_warps=8)
# The fused MLP boundary's launch (64 rows per workgroup of 4 wavefronts),
# also a valid launch of the fused residual norm at the attention boundary.
HIP_MLP_BOUNDARY_LAUNCH = NormLaunchParams(block_rows=64, num_warps=4)
# The launch of the HIP packed-QKV projection with the head-major epilogue
# (csrc/linear_gelu.hip, sah_qkv_projection): the same GEMM core.
HIP_QKV_LAUNCH = QKVLaunchParams(block_m=256, block_n=256, block_k=64, num_warps=8)


def hip_linear_boundary_launch(d_model: int) -> NormLaunchParams:
    """The launch of the HIP Linear + residual + LayerNorm boundary
    (csrc/linear_norm.hip) for a model width: 65536 / d_model whole rows per
    workgroup of 8 wavefronts."""

    return NormLaunchParams(block_rows=max(1, 65536 // d_model), num_warps=8)


def hip_config(
    *,
    microbatch_size: int | None = None,
    graph: bool = False,
    attention_launch: AttentionLaunchParams = HIP_DEFAULT_ATTENTION_LAUNCH,
    norm_launch: NormLaunchParams = HIP_DEFAULT_NORM_LAUNCH,
    ffn: FFNBackend = FFNBackend.HIP_EXACT_GELU,
    qkv: QKVMaterialization = QKVMaterialization.VIEW,
    residual_norm: ResidualNormBackend = ResidualNormBackend.HIP_FUSED,
    boundary_launch: NormLaunchParams | None = None,
    initial_norm: InitialNormBackend = InitialNormBackend.HIP,
) -> ConfigSpec:
    """The gfx950 program for 16-bit models: HIP attention, HIP fused residual
    norms and HIP initial norm, projections in the model dtype on hipBLASLt,
    the FFN activation by the HIP exact-GELU kernel.  ``microbatch_size`` selects the streamed schedule, ``graph``
    the graph-replay runtime (one HIP graph per input signature).  ``ffn``
    picks the FFN activation path: TORCH (hipBLASLt, then torch's exact GELU),
    HIP_EXACT_GELU (hipBLASLt, then the HIP elementwise GELU),
    HIP_LINEAR_EXACT_GELU (the fused HIP Linear + bias + exact GELU) or
    HIP_FUSED_MLP_BOUNDARY (the whole FFN and its residual LayerNorm in one
    kernel, widths 128 and 256; its launch HIP_MLP_BOUNDARY_LAUNCH is also the
    attention boundary's norm launch).  ``qkv``
    picks how Q, K and V are produced: VIEW (hipBLASLt packed projection and
    zero-copy views) or HIP_NATIVE_BHSD (the HIP projection writing
    head-major Q / K and a seq-contiguous V straight from its epilogue).
    ``residual_norm`` picks the boundary: HIP_FUSED (residual + norm after the
    hipBLASLt output projections, with ``norm_launch``) or HIP_LINEAR_FUSED
    (each output projection fused into its boundary, with ``boundary_launch``,
    see hip_linear_boundary_launch).  ``initial_norm`` picks the layer-0
    LayerNorm: HIP (its own kernel, with ``norm_launch``) or HIP_FUSED_QKV
    (fused into the HIP_NATIVE_BHSD projection, which it requires)."""

    ffn = FFNBackend(ffn)
    if ffn not in {
        FFNBackend.TORCH,
        FFNBackend.HIP_EXACT_GELU,
        FFNBackend.HIP_LINEAR_EXACT_GELU,
        FFNBackend.HIP_FUSED_MLP_BOUNDARY,
    }:
        raise ValueError(f"FFN backend {ffn.value!r} is not part of the gfx950 program")
    qkv = QKVMaterialization(qkv)
    if qkv not in {QKVMaterialization.VIEW, QKVMaterialization.HIP_NATIVE_BHSD}:
        raise ValueError(f"QKV materialization {qkv.value!r} is not part of the gfx950 program")
    initial_norm = InitialNormBackend(initial_norm)
    if initial_norm not in {InitialNormBackend.HIP, InitialNormBackend.HIP_FUSED_QKV}:
        raise ValueError(f"initial norm {initial_norm.value!r} is not part of the gfx950 program")
    if initial_norm is InitialNormBackend.HIP_FUSED_QKV and qkv is not QKVMaterialization.HIP_NATIVE_BHSD:
        raise ValueError("the fused initial norm runs inside the HIP_NATIVE_BHSD QKV projection")
    residual_norm = ResidualNormBackend(residual_norm)
    if residual_norm is ResidualNormBackend.HIP_LINEAR_FUSED:
        if boundary_launch is None:
            raise ValueError("the linear boundary needs boundary_launch (hip_linear_boundary_launch(d_model))")
        residual_launch = boundary_launch
    elif residual_norm is ResidualNormBackend.HIP_FUSED:
        if boundary_launch is not None:
            raise ValueError("boundary_launch is only for the linear boundary")
        # the fused MLP boundary runs with the residual-norm launch
        residual_launch = HIP_MLP_BOUNDARY_LAUNCH if ffn is FFNBackend.HIP_FUSED_MLP_BOUNDARY else norm_launch
    else:
        raise ValueError(f"residual norm {residual_norm.value!r} is not part of the gfx950 program")
    if ffn is FFNBackend.HIP_FUSED_MLP_BOUNDARY and residual_norm is not ResidualNormBackend.HIP_FUSED:
        raise ValueError("the fused MLP boundary pairs with the HIP_FUSED attention boundary")

    if graph and microbatch_size is not None:
        raise ValueError("the graph runtime and the streamed schedule are exclusive")
    if graph:
        runtime = RuntimeBackend.CUDA_GRAPH
    else:
        runtime = RuntimeBackend.EAGER if microbatch_size is None else RuntimeBackend.STREAMED
    return ConfigSpec(
        program=ProgramConfig(
            attention=AttentionBackend.HIP_STREAMING_DH64,
            qkv_projection=ProjectionBackend.INPUT_DTYPE,
            attention_output_projection=ProjectionBackend.INPUT_DTYPE,
            ffn_input_projection=ProjectionBackend.INPUT_DTYPE,
            ffn_output_projection=ProjectionBackend.INPUT_DTYPE,
            precision_plan=PrecisionPlan.INPUT_DTYPE,
            qkv_materialization=qkv,
            attention_output_bridge=AttentionOutputBridge.ATTENTION_DIRECT_BSD,
            ffn=ffn,
            residual_norm=residual_norm,
            initial_norm=initial_norm,
        ),
        schedule=ScheduleConfig(
            runtime=runtime,
            attention_launch=attention_launch,
            qkv_launch=HIP_QKV_LAUNCH if qkv is QKVMaterialization.HIP_NATIVE_BHSD else None,
            residual_norm_launch=residual_launch,
            initial_norm_launch=norm_launch if initial_norm is InitialNormBackend.HIP else None,
            ffn_launch=HIP_GELU_LAUNCH if ffn is FFNBackend.HIP_EXACT_GELU else None,
            ffn_input_launch=HIP_LINEAR_LAUNCH if ffn is FFNBackend.HIP_LINEAR_EXACT_GELU else None,
            microbatch_size=microbatch_size,
        ),
    )


__all__ = [
    "COMPILED_FORWARD_MODES",
    "CONFIG_SCHEMA_VERSION",
    "DEFAULT_COMPILED_FORWARD_MODE",
    "DIRECT_BSD_ATTENTION_BACKENDS",
    "HIP_ATTENTION_BACKENDS",
    "HIP_DEFAULT_ATTENTION_LAUNCH",
    "HIP_DEFAULT_NORM_LAUNCH",
    "HIP_GELU_LAUNCH",
    "HIP_MLP_BOUNDARY_LAUNCH",
    "HIP_LINEAR_LAUNCH",
    "HIP_QKV_LAUNCH",
    "HIP_LONG_SEQUENCE_ATTENTION_LAUNCH",
    "HIP_RESIDUAL_NORM_BACKENDS",
    "LINEAR_BOUNDARY_RESIDUAL_NORM_BACKENDS",
    "hip_linear_boundary_launch",
    "LAUNCHED_ATTENTION_BACKENDS",
    "NATIVE_QKV_MATERIALIZATIONS",
    "TRITON_ATTENTION_BACKENDS",
    "AttentionBackend",
    "AttentionLaunchParams",
    "AttentionOutputBridge",
    "AttentionOutputLayout",
    "ConfigSpec",
    "FFNBackend",
    "FFNLaunchParams",
    "GemmLaunchParams",
    "InitialNormBackend",
    "NormLaunchParams",
    "PrecisionPlan",
    "ProgramConfig",
    "ProjectionBackend",
    "QKVLaunchParams",
    "QKVMaterialization",
    "ResidualNormBackend",
    "RuntimeBackend",
    "ScheduleConfig",
    "TritonAttentionParams",
    "TritonFFNParams",
    "TritonGemmParams",
    "TritonNormParams",
    "TritonQKVParams",
    "fp16_projection_fields",
    "hip_config",
    "portable_config",
    "portable_streamed_config",
]
