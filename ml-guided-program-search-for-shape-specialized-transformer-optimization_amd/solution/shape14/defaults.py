"""Default streamed programs.

conservative_streamed_config restates the reference's measured low-risk
Shape 14 program (solution/shape14/defaults.py:22-49) so its config_id can be
reproduced; its Triton attention is rejected by this build's PlanBuilder.

hip_streamed_config is the gfx950 program for long sequences: HIP streaming
attention (256-row tiles over 8 wavefronts) and HIP norms with ordered
microbatches (2 sequences per chunk by default, the BASELINE long-sequence
configuration).

hip_deployed_shape14_config is the reference's deployed long-sequence
program for fp32 models (deployment/deployed_configs.json:774-822: fp32 I/O,
fp16 QKV / attention-output / FFN-input projections, fp16 streaming
attention, fp32 GELU and FFN output projection, fp32 norms) with the HIP
attention and the HIP fp32 norms in place of its Triton and torch ones.

hip_mixed_streamed_config is the fp32-model program with fp16 branches
throughout: every projection in fp16 and the HIP mixed residual norms (fp32
stream, fp16 update and normalized output).
"""

from __future__ import annotations

from solution.config import (
    HIP_DEFAULT_NORM_LAUNCH,
    HIP_LONG_SEQUENCE_ATTENTION_LAUNCH,
    AttentionBackend,
    AttentionLaunchParams,
    AttentionOutputBridge,
    ConfigSpec,
    FFNBackend,
    InitialNormBackend,
    NormLaunchParams,
    PrecisionPlan,
    ProgramConfig,
    ProjectionBackend,
    QKVMaterialization,
    ResidualNormBackend,
    RuntimeBackend,
    ScheduleConfig,
    hip_config,
)

DEFAULT_MICROBATCH_SIZE = 2


def conservative_streamed_config() -> ConfigSpec:
    """The reference's pre-tuning Shape 14 program (Triton attention)."""

    return ConfigSpec(
        program=ProgramConfig(
            attention=AttentionBackend.TRITON_STREAMING_DH64,
            qkv_projection=ProjectionBackend.FP16_SHADOW,
            attention_output_projection=ProjectionBackend.FP16_SHADOW,
            ffn_input_projection=ProjectionBackend.FP16_SHADOW,
            ffn_output_projection=ProjectionBackend.INPUT_DTYPE,
            precision_plan=PrecisionPlan.FP16_ATTENTION_AND_FFN_INPUT,
            qkv_materialization=QKVMaterialization.VIEW,
            attention_output_bridge=AttentionOutputBridge.ATTENTION_DIRECT_BSD,
            ffn=FFNBackend.TORCH,
            residual_norm=ResidualNormBackend.TORCH,
            initial_norm=InitialNormBackend.TORCH,
        ),
        schedule=ScheduleConfig(
            runtime=RuntimeBackend.STREAMED,
            attention_launch=AttentionLaunchParams(block_m=32, block_n=64, num_warps=4, num_stages=2),
            microbatch_size=1,
        ),
    )


def hip_streamed_config(
    *,
    microbatch_size: int = DEFAULT_MICROBATCH_SIZE,
    ffn: FFNBackend = FFNBackend.HIP_EXACT_GELU,
    qkv: QKVMaterialization = QKVMaterialization.VIEW,
    residual_norm: ResidualNormBackend = ResidualNormBackend.HIP_FUSED,
    boundary_launch: NormLaunchParams | None = None,
    initial_norm: InitialNormBackend = InitialNormBackend.HIP,
) -> ConfigSpec:
    """The gfx950 long-sequence program with ordered microbatches."""

    return hip_config(
        microbatch_size=microbatch_size,
        attention_launch=HIP_LONG_SEQUENCE_ATTENTION_LAUNCH,
        ffn=ffn,
        qkv=qkv,
        residual_norm=residual_norm,
        boundary_launch=boundary_launch,
        initial_norm=initial_norm,
    )


def hip_deployed_shape14_config(*, microbatch_size: int = DEFAULT_MICROBATCH_SIZE) -> ConfigSpec:
    """The reference's deployed Shape 14 program for fp32 models
    (FP16_ATTENTION_AND_FFN_INPUT: fp16 shadow QKV, attention-output and
    FFN-input projections, fp32 GELU and FFN output projection) with the HIP
    fp16 streaming attention and the HIP fp32 residual / initial norms, with
    ordered microbatches."""

    return ConfigSpec(
        program=ProgramConfig(
            attention=AttentionBackend.HIP_STREAMING_DH64,
            qkv_projection=ProjectionBackend.FP16_SHADOW,
            attention_output_projection=ProjectionBackend.FP16_SHADOW,
            ffn_input_projection=ProjectionBackend.FP16_SHADOW,
            ffn_output_projection=ProjectionBackend.INPUT_DTYPE,
            precision_plan=PrecisionPlan.FP16_ATTENTION_AND_FFN_INPUT,
            qkv_materialization=QKVMaterialization.VIEW,
            attention_output_bridge=AttentionOutputBridge.ATTENTION_DIRECT_BSD,
            ffn=FFNBackend.TORCH,
            residual_norm=ResidualNormBackend.HIP_FUSED,
            initial_norm=InitialNormBackend.HIP,
        ),
        schedule=ScheduleConfig(
            runtime=RuntimeBackend.STREAMED,
            attention_launch=HIP_LONG_SEQUENCE_ATTENTION_LAUNCH,
            residual_norm_launch=HIP_DEFAULT_NORM_LAUNCH,
            initial_norm_launch=HIP_DEFAULT_NORM_LAUNCH,
            microbatch_size=microbatch_size,
        ),
    )


def hip_mixed_streamed_config(*, microbatch_size: int = DEFAULT_MICROBATCH_SIZE) -> ConfigSpec:
    """fp32 models: fp32 residual stream, every projection on FP16 shadow
    weights, fp16 HIP streaming attention, the HIP mixed residual norms
    (fp32 residual + fp16 update -> fp32 residual, fp16 normalized; fp32 at the
    final boundary), the HIP initial norm and torch's exact GELU, with ordered
    microbatches.  The reference's deployed program keeps the FFN output
    projection in fp32 with torch norms; the mixed HIP norm takes the fp16
    FFN update instead (its FP16_CORE precision plan)."""

    return ConfigSpec(
        program=ProgramConfig(
            attention=AttentionBackend.HIP_STREAMING_DH64,
            qkv_projection=ProjectionBackend.FP16_SHADOW,
            attention_output_projection=ProjectionBackend.FP16_SHADOW,
            ffn_input_projection=ProjectionBackend.FP16_SHADOW,
            ffn_output_projection=ProjectionBackend.FP16_SHADOW,
            precision_plan=PrecisionPlan.FP16_CORE,
            qkv_materialization=QKVMaterialization.VIEW,
            attention_output_bridge=AttentionOutputBridge.ATTENTION_DIRECT_BSD,
            ffn=FFNBackend.TORCH,
            residual_norm=ResidualNormBackend.HIP_MIXED,
            initial_norm=InitialNormBackend.HIP,
        ),
        schedule=ScheduleConfig(
            runtime=RuntimeBackend.STREAMED,
            attention_launch=HIP_LONG_SEQUENCE_ATTENTION_LAUNCH,
            residual_norm_launch=HIP_DEFAULT_NORM_LAUNCH,
            initial_norm_launch=HIP_DEFAULT_NORM_LAUNCH,
            microbatch_size=microbatch_size,
        ),
    )


__all__ = [
    "DEFAULT_MICROBATCH_SIZE",
    "conservative_streamed_config",
    "hip_deployed_shape14_config",
    "hip_mixed_streamed_config",
    "hip_streamed_config",
]
