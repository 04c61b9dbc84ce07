"""Plan API: config format and ids, legality, streamed schedule (CPU only)."""

from __future__ import annotations

import dataclasses
import json
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from solution.config import (
    AttentionBackend,
    AttentionLaunchParams,
    ConfigSpec,
    FFNBackend,
    InitialNormBackend,
    NormLaunchParams,
    ProgramConfig,
    ResidualNormBackend,
    RuntimeBackend,
    ScheduleConfig,
    TritonAttentionParams,
    hip_config,
    portable_config,
)
from solution.plan import ExecutionContext
from solution.plan_builder import ConfigRejectedError, HardwareCapabilities, PlanBuilder
from solution.shape14.defaults import conservative_streamed_config, hip_streamed_config
from solution.shape14.executor import execute_streamed
from solution.transformer import _is_official_shape14, _uses_streamed_scope

GOLDEN = Path(__file__).resolve().parent / "golden"


def _gfx950(**overrides) -> HardwareCapabilities:
    values = dict(
        device_type="cuda",
        compute_capability=(9, 5),
        shared_memory_per_block=65536,
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
        gcn_arch="gfx950",
        hip_streaming_dh64_attention=True,
        hip_residual_norm=True,
        hip_initial_norm=True,
        hip_linear_exact_gelu=True,
        hip_exact_gelu=True,
        hip_qkv_native_bhsd=True,
        hip_linear_residual_norm=True,
        hip_mlp_residual_norm=True,
    )
    values.update(overrides)
    return HardwareCapabilities(**values)


def _context(batch=32, seq=100000, d=1024, heads=16, ffn=4096, layers=2, *, dtype=torch.bfloat16,
             device="cuda", mask=False, grad=False) -> ExecutionContext:
    return ExecutionContext(
        batch_size=batch,
        seq_len=seq,
        d_model=d,
        num_heads=heads,
        causal=True,
        device=torch.device(device),
        dtype=dtype,
        training=False,
        grad_enabled=grad,
        input_contiguous=True,
        has_valid_token_mask=mask,
        mask_compatible=True,
        ffn_dim=ffn,
        num_layers=layers,
    )


# ---------------------------------------------------------------- config ids


def test_reference_config_ids_are_reproduced():
    """Golden ids: tests/benchmarking/test_shape14_defaults.py:12-13 and the
    deployed Shape 14 program (final_performance.json:407) of the reference."""

    assert conservative_streamed_config().config_id == (
        "cfg-3d94f979e8424ea78bfd0656a0d32182cb9f0e706f85b805e6d01571496b75ec"
    )
    assert conservative_streamed_config().schedule.attention_launch.to_dict() == {
        "block_m": 32, "block_n": 64, "num_warps": 4, "num_stages": 2,
    }


def test_every_reference_deployed_config_round_trips_with_its_published_id():
    records = json.loads((GOLDEN / "reference_configs.json").read_text())["records"]
    assert len(records) == 14
    for record in records:
        config = ConfigSpec.from_dict(record["config"])
        assert config.to_dict() == record["config"]
        assert config.config_id == record["published_config_id"], record["case_id"]
    shape14 = ConfigSpec.from_dict(records[-1]["config"])
    assert shape14.config_id == "cfg-cc77d6b483e1f07e137d89773db64dd8a3367f901dbae918aa7cebffd405ab60"


def test_canonical_json_is_sorted_compact_ascii():
    text = portable_config().canonical_json()
    assert " " not in text and text.isascii()
    assert text == json.dumps(json.loads(text), sort_keys=True, separators=(",", ":"))
    assert portable_config().config_id == "cfg-" + portable_config().sha256


def test_hip_config_round_trips_and_uses_existing_fields():
    config = hip_config(microbatch_size=2)
    payload = config.to_dict()
    assert set(payload["schedule"]) == set(portable_config().to_dict()["schedule"])
    assert ConfigSpec.from_dict(json.loads(json.dumps(payload))) == config
    assert payload["program"]["attention"] == "hip_streaming_dh64"
    assert payload["program"]["residual_norm"] == "hip_fused"
    assert payload["program"]["initial_norm"] == "hip"
    streamed = hip_streamed_config()
    assert streamed.schedule.attention_launch == AttentionLaunchParams(256, 64, 8, 2)
    assert streamed == hip_config(microbatch_size=2, attention_launch=streamed.schedule.attention_launch)
    assert TritonAttentionParams is AttentionLaunchParams


def test_presence_rules_cover_hip_backends():
    program = hip_config().program
    with pytest.raises(ValueError, match="attention_launch"):
        ConfigSpec(program=program, schedule=ScheduleConfig(runtime=RuntimeBackend.EAGER))
    with pytest.raises(ValueError, match="residual_norm_launch"):
        ConfigSpec(
            program=program,
            schedule=ScheduleConfig(
                runtime=RuntimeBackend.EAGER,
                attention_launch=AttentionLaunchParams(128, 64, 4, 2),
                initial_norm_launch=NormLaunchParams(4, 4),
            ),
        )


@pytest.mark.parametrize(
    "field,payload",
    [
        ("attention_launch", {"block_m": 96, "block_n": 64, "num_warps": 4, "num_stages": 2}),
        ("attention_launch", {"block_m": 128, "block_n": 64, "num_warps": 3, "num_stages": 2}),
        ("attention_launch", {"block_m": 128, "block_n": 64, "num_warps": 4}),
        ("residual_norm_launch", {"block_rows": 4, "num_warps": 4, "extra": 1}),
    ],
)
def test_launch_objects_are_exact_and_validated(field, payload):
    document = hip_config().to_dict()
    document["schedule"][field] = payload
    with pytest.raises((ValueError, TypeError)):
        ConfigSpec.from_dict(document)


# ---------------------------------------------------------------- legality


def test_hip_plan_is_accepted_for_the_long_sequence_configuration():
    plan = PlanBuilder().build(hip_streamed_config(), _context(), _gfx950())
    assert plan.use_streamed_execution
    assert plan.inner_context.batch_size == 2 and plan.outer_context.batch_size == 32
    assert plan.attention_compute_dtype == "bfloat16"
    trace = plan.expected_trace.to_dict()
    assert trace["attention_calls"] == 2 and trace["residual_norm_calls"] == 4
    assert trace["initial_norm_calls"] == 1 and trace["complete"] is True
    description = plan.describe()
    assert description["causal_mask"] == "online_causal"
    assert description["inner_batch_size"] == 2


def test_hip_plan_rejections_are_structured():
    builder = PlanBuilder()
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    cpu = builder.evaluate(hip_config(), _context(device="cpu"), _gfx950(device_type="cpu", gcn_arch=None))
    assert ("program.attention", "requires_cuda") in codes(cpu)
    mi300 = builder.evaluate(hip_config(), _context(), _gfx950(gcn_arch="gfx942"))
    assert ("program.attention", "requires_gfx950") in codes(mi300)
    wide_heads = builder.evaluate(hip_config(), _context(heads=8), _gfx950())
    assert ("program.attention", "unsupported_shape") in codes(wide_heads)
    # fp32 models: HIP attention (the fp32 kernel) and HIP norms, torch's FFN
    # activation; the 16-bit elementwise GELU kernel rejects the fp32 context
    fp32 = builder.evaluate(hip_config(ffn=FFNBackend.TORCH), _context(dtype=torch.float32), _gfx950())
    assert not fp32.violations, fp32.violations
    fp32_gelu = builder.evaluate(hip_config(), _context(dtype=torch.float32), _gfx950())
    assert ("program.ffn", "unsupported_dtype") in codes(fp32_gelu)
    assert not any(field == "program.qkv_projection" for field, _ in codes(fp32_gelu))
    missing = builder.evaluate(hip_config(), _context(), _gfx950(hip_streaming_dh64_attention=False,
                                                                  hip_residual_norm=False))
    assert ("program.attention", "backend_unavailable") in codes(missing)
    assert ("program.residual_norm", "backend_unavailable") in codes(missing)
    grad = builder.evaluate(hip_config(), _context(grad=True), _gfx950())
    assert ("program.attention", "requires_inference") in codes(grad)
    odd_width = builder.evaluate(hip_config(), _context(d=1000, heads=10), _gfx950())
    assert ("program.residual_norm", "unsupported_shape") in codes(odd_width)
    with pytest.raises(ConfigRejectedError, match="program.attention"):
        builder.build(hip_config(), _context(heads=8), _gfx950())


def test_streamed_microbatch_rules():
    builder = PlanBuilder()
    for batch, microbatch, code in ((6, 4, "microbatch_not_divisor"), (2, 4, "microbatch_exceeds_batch")):
        result = builder.evaluate(hip_config(microbatch_size=microbatch), _context(batch=batch), _gfx950())
        assert ("schedule.microbatch_size", code) in {(v.field, v.code) for v in result.violations}
    masked = builder.evaluate(hip_config(microbatch_size=2), _context(mask=True), _gfx950())
    assert ("schedule.runtime", "mask_not_supported") in {(v.field, v.code) for v in masked.violations}


def test_graph_runtime_plans_for_inference_on_the_gpu():
    builder = PlanBuilder()
    config = hip_config(graph=True)
    assert config.schedule.runtime is RuntimeBackend.CUDA_GRAPH
    assert ConfigSpec.from_dict(json.loads(json.dumps(config.to_dict()))) == config
    short = _context(batch=64, seq=256, d=512, heads=8, ffn=2048, layers=4)
    plan = builder.build(config, short, _gfx950())
    assert plan.use_cuda_graph and plan.describe()["runtime_backend"] == "cuda_graph"
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    cpu = builder.evaluate(config, _context(device="cpu"), _gfx950(device_type="cpu", gcn_arch=None))
    assert ("schedule.runtime", "requires_cuda") in codes(cpu)
    grad = builder.evaluate(config, _context(grad=True), _gfx950())
    assert ("schedule.runtime", "requires_inference") in codes(grad)
    with pytest.raises(ValueError, match="exclusive"):
        hip_config(graph=True, microbatch_size=2)


def test_reference_only_backends_are_unavailable_not_silently_replaced():
    records = json.loads((GOLDEN / "reference_configs.json").read_text())["records"]
    builder = PlanBuilder()
    shape14 = ConfigSpec.from_dict(records[-1]["config"])
    result = builder.evaluate(shape14, _context(dtype=torch.float32, ffn=1024), _gfx950())
    assert not result.accepted
    assert ("program.attention", "backend_unavailable") in {(v.field, v.code) for v in result.violations}
    # the reference's deployed Shape 14 program with only the attention swapped is legal
    program = ProgramConfig.from_dict({**records[-1]["config"]["program"], "attention": "hip_streaming_dh64"})
    schedule = dataclasses.replace(shape14.schedule, attention_launch=AttentionLaunchParams(128, 64, 4, 2))
    swapped = ConfigSpec(program=program, schedule=schedule)
    plan = builder.build(swapped, _context(dtype=torch.float32, ffn=1024), _gfx950())
    assert plan.attention_compute_dtype == "float16"  # FP16 shadow QKV feeds the HIP kernel


def test_portable_configs_are_legal_on_cpu():
    cpu = _gfx950(device_type="cpu", gcn_arch=None, hip_streaming_dh64_attention=False)
    plan = PlanBuilder().build(portable_config(), _context(batch=2, seq=16, d=64, heads=4, device="cpu",
                                                           dtype=torch.float32), cpu)
    assert plan.attention_backend is AttentionBackend.REFERENCE_STREAMING
    assert plan.describe()["causal_mask"] == "query_block"


def test_mixed_stream_plan_requires_fp16_updates():
    program = ProgramConfig(
        attention=AttentionBackend.HIP_STREAMING_DH64,
        qkv_projection="fp16_shadow",
        attention_output_projection="fp16_shadow",
        ffn_input_projection="fp16_shadow",
        ffn_output_projection="fp16_shadow",
        precision_plan="fp16_core",
        qkv_materialization="view",
        attention_output_bridge="attention_direct_bsd",
        ffn="torch",
        residual_norm=ResidualNormBackend.HIP_MIXED,
        initial_norm=InitialNormBackend.HIP,
    )
    schedule = ScheduleConfig(
        runtime=RuntimeBackend.EAGER,
        attention_launch=AttentionLaunchParams(128, 64, 4, 2),
        residual_norm_launch=NormLaunchParams(4, 4),
        initial_norm_launch=NormLaunchParams(4, 4),
    )
    plan = PlanBuilder().build(ConfigSpec(program=program, schedule=schedule),
                               _context(dtype=torch.float32), _gfx950())
    assert plan.use_mixed_residual_stream
    bf16 = PlanBuilder().evaluate(ConfigSpec(program=program, schedule=schedule), _context(), _gfx950())
    assert ("program.residual_norm", "requires_float32_input") in {(v.field, v.code) for v in bf16.violations}


# ------------------------------------------------------------ streamed driver


def test_official_shape14_and_long_sequences_use_the_streamed_scope():
    """Restates tests/solution/test_shape14_isolation.py:18-27 of the reference
    and adds the F=4096 long-sequence configuration."""

    config = SimpleNamespace(num_heads=16, num_layers=2, ffn_dim=1024, causal=True)
    assert _is_official_shape14(config, (32, 100000, 1024))
    assert not _is_official_shape14(config, (1, 100000, 1024))
    wide = SimpleNamespace(num_heads=16, num_layers=2, ffn_dim=4096, causal=True)
    assert _uses_streamed_scope(wide, (32, 100000, 1024))
    assert not _uses_streamed_scope(wide, (64, 256, 512))


def test_streamed_executor_preserves_order_and_mask_slices():
    """Restates tests/solution/test_shape14_isolation.py:56-89."""

    value = torch.arange(24, dtype=torch.float32).reshape(4, 3, 2)
    mask = torch.tensor([[True, True, True], [True, False, False], [True, True, False], [False, False, False]])
    seen: list[torch.Tensor] = []

    def forward_chunk(chunk, chunk_mask):
        seen.append(chunk_mask.clone())
        return chunk + 1

    output = execute_streamed(value, mask, microbatch_size=2, forward_chunk=forward_chunk)
    torch.testing.assert_close(output, value + 1)
    torch.testing.assert_close(torch.cat(seen), mask)


@pytest.mark.parametrize("microbatch_size", [0, True, 3])
def test_streamed_executor_rejects_invalid_microbatches(microbatch_size):
    with pytest.raises(ValueError):
        execute_streamed(torch.zeros(4, 2, 1), None, microbatch_size=microbatch_size,
                         forward_chunk=lambda chunk, mask: chunk)


def test_streamed_executor_writes_chunks_into_the_preallocated_output():
    value = torch.arange(32, dtype=torch.float32).reshape(8, 2, 2)
    destinations: list[int] = []

    def forward_chunk(chunk, mask, destination):
        destinations.append(destination.data_ptr())
        torch.mul(chunk, 2, out=destination)
        return destination

    output = execute_streamed(value, None, microbatch_size=2, forward_chunk=forward_chunk,
                              write_into_output=True)
    assert torch.equal(output, value * 2)
    assert destinations == [output[i:i + 2].data_ptr() for i in range(0, 8, 2)]
    copied = execute_streamed(value, None, microbatch_size=4,
                              forward_chunk=lambda chunk, mask, destination: chunk - 1,
                              write_into_output=True)
    assert torch.equal(copied, value - 1)


def test_fused_ffn_input_plans_and_rejections():
    """The HIP Linear + exact-GELU FFN backend: accepted for 16-bit inference on
    gfx950 with its launch, rejected with structured reasons otherwise (the
    reference's TRITON_LINEAR_EXACT_GELU rules, solution/plan_builder.py:825-866)."""

    import dataclasses

    from solution.config import FFNBackend, GemmLaunchParams, PrecisionPlan

    builder = PlanBuilder()
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    fused = hip_config(ffn=FFNBackend.HIP_LINEAR_EXACT_GELU)
    assert fused.program.ffn is FFNBackend.HIP_LINEAR_EXACT_GELU
    assert fused.schedule.ffn_input_launch == GemmLaunchParams(256, 256, 64, 8, 2)
    assert ConfigSpec.from_dict(fused.to_dict()) == fused
    plan = builder.build(fused, _context(batch=64, seq=256, d=512, heads=8, ffn=2048, layers=4), _gfx950())
    assert plan.ffn_backend is FFNBackend.HIP_LINEAR_EXACT_GELU
    assert plan.expected_trace.to_dict()["ffn_activation_output_dtype"] == "bfloat16"
    streamed = builder.build(hip_streamed_config(ffn=FFNBackend.HIP_LINEAR_EXACT_GELU), _context(), _gfx950())
    assert streamed.use_streamed_execution and streamed.ffn_input_launch is not None
    # the launch is part of the schedule exactly when the fused backend is selected
    with pytest.raises(ValueError, match="ffn_input_launch"):
        dataclasses.replace(fused, schedule=dataclasses.replace(fused.schedule, ffn_input_launch=None))
    unavailable = builder.evaluate(fused, _context(), _gfx950(hip_linear_exact_gelu=False))
    assert ("program.ffn", "backend_unavailable") in codes(unavailable)
    odd_ffn = builder.evaluate(fused, _context(ffn=4000), _gfx950())
    assert ("program.ffn", "unsupported_shape") in codes(odd_ffn)
    wrong_launch = dataclasses.replace(
        fused, schedule=dataclasses.replace(fused.schedule, ffn_input_launch=GemmLaunchParams(128, 128, 32, 4, 2))
    )
    assert ("schedule.ffn_input_launch", "unsupported_launch_value") in codes(builder.evaluate(wrong_launch, _context(), _gfx950()))
    # an fp32-GELU precision plan needs FP16 projections, which the fused
    # backend does not multiply: the program itself is invalid
    with pytest.raises(ValueError, match="FP16 backend"):
        dataclasses.replace(fused.program, precision_plan=PrecisionPlan.FP16_FFN_INPUT_FP32_GELU)
    training = builder.evaluate(fused, _context(grad=True), _gfx950())
    assert ("program.ffn", "requires_inference") in codes(training)


def test_elementwise_gelu_plans_and_rejections():
    """The HIP elementwise exact GELU after the hipBLASLt input projection
    (the reference's TRITON_EXACT_GELU rules, solution/plan_builder.py:870-900,
    for 16-bit models)."""

    import dataclasses

    from solution.config import FFNBackend, FFNLaunchParams

    builder = PlanBuilder()
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    gelu = hip_config(ffn=FFNBackend.HIP_EXACT_GELU)
    assert gelu.schedule.ffn_launch == FFNLaunchParams(4096, 8) and gelu.schedule.ffn_input_launch is None
    assert hip_config() == gelu  # the default gfx950 program
    assert ConfigSpec.from_dict(gelu.to_dict()) == gelu
    plan = builder.build(gelu, _context(), _gfx950())
    assert plan.ffn_backend is FFNBackend.HIP_EXACT_GELU and plan.ffn_launch == FFNLaunchParams(4096, 8)
    with pytest.raises(ValueError, match="ffn_launch"):
        dataclasses.replace(gelu, schedule=dataclasses.replace(gelu.schedule, ffn_launch=None))
    bad_launch = dataclasses.replace(gelu, schedule=dataclasses.replace(gelu.schedule, ffn_launch=FFNLaunchParams(256, 4)))
    assert ("schedule.ffn_launch", "unsupported_launch_value") in codes(builder.evaluate(bad_launch, _context(), _gfx950()))
    unavailable = builder.evaluate(gelu, _context(), _gfx950(hip_exact_gelu=False))
    assert ("program.ffn", "backend_unavailable") in codes(unavailable)
    with pytest.raises(ValueError, match="not part of the gfx950 program"):
        hip_config(ffn=FFNBackend.TRITON_EXACT_GELU)


def test_native_qkv_plans_and_rejections():
    """The HIP native-layout QKV projection: accepted for 16-bit inference on
    gfx950 with its launch, rejected with structured reasons otherwise (the
    reference's TRITON_NATIVE_BHSD rules, solution/plan_builder.py:381-446)."""

    import dataclasses

    from solution.config import (
        HIP_QKV_LAUNCH,
        PrecisionPlan,
        ProjectionBackend,
        QKVLaunchParams,
        QKVMaterialization,
        RuntimeBackend,
    )

    builder = PlanBuilder()
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    native = hip_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD)
    assert native.program.qkv_materialization is QKVMaterialization.HIP_NATIVE_BHSD
    assert native.schedule.qkv_launch == HIP_QKV_LAUNCH == QKVLaunchParams(256, 256, 64, 8)
    assert ConfigSpec.from_dict(native.to_dict()) == native
    assert native.config_id != hip_config().config_id
    plan = builder.build(native, _context(batch=64, seq=256, d=512, heads=8, ffn=2048, layers=4), _gfx950())
    assert plan.qkv_materialization is QKVMaterialization.HIP_NATIVE_BHSD
    assert plan.expected_trace.to_dict()["qkv_materialization"] == "hip_native_bhsd"
    streamed = builder.build(hip_streamed_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD), _context(), _gfx950())
    assert streamed.use_streamed_execution and streamed.qkv_launch == HIP_QKV_LAUNCH
    # the launch is part of the schedule exactly when a native materialization is selected
    with pytest.raises(ValueError, match="qkv_launch"):
        dataclasses.replace(native, schedule=dataclasses.replace(native.schedule, qkv_launch=None))
    with pytest.raises(ValueError, match="qkv_launch"):
        dataclasses.replace(hip_config(), schedule=dataclasses.replace(hip_config().schedule, qkv_launch=HIP_QKV_LAUNCH))
    with pytest.raises(ValueError, match="not part of the gfx950 program"):
        hip_config(qkv=QKVMaterialization.CONTIGUOUS)
    unavailable = builder.evaluate(native, _context(), _gfx950(hip_qkv_native_bhsd=False))
    assert ("program.qkv_materialization", "backend_unavailable") in codes(unavailable)
    not_gfx950 = builder.evaluate(native, _context(), _gfx950(gcn_arch="gfx942"))
    assert ("program.qkv_materialization", "requires_gfx950") in codes(not_gfx950)
    odd_width = builder.evaluate(native, _context(d=640, heads=10, ffn=2560), _gfx950())
    assert ("program.qkv_materialization", "unsupported_shape") in codes(odd_width)
    fp32 = builder.evaluate(native, _context(dtype=torch.float32), _gfx950())
    assert ("program.qkv_materialization", "unsupported_dtype") in codes(fp32)
    shadow = dataclasses.replace(
        native,
        program=dataclasses.replace(
            native.program,
            precision_plan=PrecisionPlan.FP16_QKV_ATTENTION,
            qkv_projection=ProjectionBackend.FP16_SHADOW,
        ),
    )
    assert ("program.qkv_projection", "backend_incompatible") in codes(builder.evaluate(shadow, _context(), _gfx950()))
    wrong_launch = dataclasses.replace(
        native, schedule=dataclasses.replace(native.schedule, qkv_launch=QKVLaunchParams(64, 32, 32, 4))
    )
    assert ("schedule.qkv_launch", "unsupported_launch_value") in codes(builder.evaluate(wrong_launch, _context(), _gfx950()))
    compiled = dataclasses.replace(
        native,
        schedule=dataclasses.replace(native.schedule, runtime=RuntimeBackend.COMPILED_FORWARD, compile_mode="max-autotune"),
    )
    assert ("schedule.runtime", "runtime_incompatible") in codes(builder.evaluate(compiled, _context(), _gfx950()))
    training = builder.evaluate(native, _context(grad=True), _gfx950())
    assert ("program.qkv_materialization", "requires_inference") in codes(training)
    # the reference's Triton materialization stays unavailable, not replaced
    triton = dataclasses.replace(
        native, program=dataclasses.replace(native.program, qkv_materialization=QKVMaterialization.TRITON_NATIVE_BHSD)
    )
    assert ("program.qkv_materialization", "backend_unavailable") in codes(builder.evaluate(triton, _context(), _gfx950()))


def test_fused_initial_norm_qkv_plans_and_rejections():
    """Layer 0's LayerNorm inside the HIP native-layout QKV projection: no
    launch of its own, the native projection required, 16-bit widths
    512-4096, no mask (the reference's TRITON_FUSED_QKV rules,
    solution/plan_builder.py:1100-1159, with this kernel's domain)."""

    from solution.config import HIP_DEFAULT_NORM_LAUNCH, QKVMaterialization

    builder = PlanBuilder()
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    fused = hip_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD, initial_norm=InitialNormBackend.HIP_FUSED_QKV)
    assert fused.program.initial_norm is InitialNormBackend.HIP_FUSED_QKV
    assert fused.schedule.initial_norm_launch is None
    assert ConfigSpec.from_dict(fused.to_dict()) == fused
    assert fused.to_dict()["program"]["initial_norm"] == "hip_fused_qkv"
    assert fused.config_id != hip_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD).config_id
    c2 = _context(batch=64, seq=256, d=512, heads=8, ffn=2048, layers=4)
    plan = builder.build(fused, c2, _gfx950())
    assert plan.use_fused_initial_norm_qkv and not plan.use_hip_initial_norm
    trace = plan.expected_trace.to_dict()
    assert trace["initial_norm_backend"] == "hip_fused_qkv" and trace["initial_norm_launch"] is None
    streamed = builder.build(
        hip_streamed_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD, initial_norm=InitialNormBackend.HIP_FUSED_QKV),
        _context(),
        _gfx950(),
    )
    assert streamed.use_streamed_execution and streamed.use_fused_initial_norm_qkv
    # presence rule: no initial_norm_launch for the fused backend
    with pytest.raises(ValueError, match="initial_norm_launch"):
        dataclasses.replace(fused, schedule=dataclasses.replace(fused.schedule, initial_norm_launch=HIP_DEFAULT_NORM_LAUNCH))
    with pytest.raises(ValueError, match="HIP_NATIVE_BHSD"):
        hip_config(initial_norm=InitialNormBackend.HIP_FUSED_QKV)
    with pytest.raises(ValueError, match="not part of the gfx950 program"):
        hip_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD, initial_norm=InitialNormBackend.TRITON_FUSED_QKV)
    # the native projection is required (a hand-edited program without it)
    viewed = dataclasses.replace(
        fused,
        program=dataclasses.replace(fused.program, qkv_materialization=QKVMaterialization.VIEW),
        schedule=dataclasses.replace(fused.schedule, qkv_launch=None),
    )
    assert ("program.initial_norm", "qkv_incompatible") in codes(builder.evaluate(viewed, c2, _gfx950()))
    odd_width = builder.evaluate(fused, _context(d=768, heads=12, ffn=3072), _gfx950())
    assert ("program.initial_norm", "unsupported_shape") in codes(odd_width)
    assert ("program.qkv_materialization", "unsupported_shape") not in codes(odd_width)
    fp32 = builder.evaluate(fused, _context(dtype=torch.float32), _gfx950())
    assert ("program.initial_norm", "unsupported_dtype") in codes(fp32)
    masked = builder.evaluate(fused, _context(mask=True), _gfx950())
    assert ("program.initial_norm", "mask_not_supported") in codes(masked)
    unavailable = builder.evaluate(fused, c2, _gfx950(hip_qkv_native_bhsd=False))
    assert ("program.initial_norm", "backend_unavailable") in codes(unavailable)
    cpu = builder.evaluate(fused, _context(device="cpu"), _gfx950())
    assert ("program.initial_norm", "requires_gfx950") in codes(cpu)
    # the reference's Triton fusion stays unavailable, not replaced
    triton = dataclasses.replace(
        fused, program=dataclasses.replace(fused.program, initial_norm=InitialNormBackend.TRITON_FUSED_QKV)
    )
    assert ("program.initial_norm", "backend_unavailable") in codes(builder.evaluate(triton, c2, _gfx950()))


def test_fused_mlp_boundary_plans_and_rejections():
    """The whole FFN fused through its residual LayerNorm (the reference's
    TRITON_FUSED_MLP_BOUNDARY rules, solution/plan_builder.py:783-800): the
    kernel's widths, native-dtype FFN weights, the launch carried by
    residual_norm_launch, paired with the HIP fused residual norm."""

    from solution.config import HIP_MLP_BOUNDARY_LAUNCH, FFNBackend, PrecisionPlan, ProjectionBackend

    builder = PlanBuilder()
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    fused = hip_config(ffn=FFNBackend.HIP_FUSED_MLP_BOUNDARY)
    assert fused.program.ffn is FFNBackend.HIP_FUSED_MLP_BOUNDARY
    assert fused.schedule.residual_norm_launch == HIP_MLP_BOUNDARY_LAUNCH == NormLaunchParams(64, 4)
    assert fused.schedule.ffn_launch is None and fused.schedule.ffn_input_launch is None
    assert ConfigSpec.from_dict(fused.to_dict()) == fused
    assert fused.to_dict()["program"]["ffn"] == "hip_fused_mlp_boundary"
    small = _context(batch=8, seq=128, d=256, heads=4, ffn=1024, layers=2)
    plan = builder.build(fused, small, _gfx950())
    assert plan.use_fused_mlp_boundary
    trace = plan.expected_trace.to_dict()
    assert trace["ffn_backend"] == "hip_fused_mlp_boundary" and trace["residual_norm_calls"] == 4
    # the reference's own width
    assert builder.build(fused, _context(batch=64, seq=128, d=128, heads=2, ffn=128, layers=2), _gfx950())
    with pytest.raises(ValueError, match="HIP_FUSED attention boundary"):
        from solution.config import ResidualNormBackend, hip_linear_boundary_launch

        hip_config(
            ffn=FFNBackend.HIP_FUSED_MLP_BOUNDARY,
            residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED,
            boundary_launch=hip_linear_boundary_launch(512),
        )
    wide = builder.evaluate(fused, _context(batch=2, seq=256, d=512, heads=8, ffn=2048), _gfx950())
    assert ("program.ffn", "unsupported_shape") in codes(wide)
    odd_ffn = builder.evaluate(fused, _context(batch=8, seq=128, d=256, heads=4, ffn=1000), _gfx950())
    assert ("program.ffn", "unsupported_shape") in codes(odd_ffn)
    fp32 = builder.evaluate(fused, _context(batch=8, seq=128, d=256, heads=4, ffn=1024, dtype=torch.float32), _gfx950())
    assert ("program.ffn", "unsupported_dtype") in codes(fp32)
    masked = builder.evaluate(fused, _context(batch=8, seq=128, d=256, heads=4, ffn=1024, mask=True), _gfx950())
    assert ("program.ffn", "mask_not_supported") in codes(masked)
    unavailable = builder.evaluate(fused, small, _gfx950(hip_mlp_residual_norm=False))
    assert ("program.ffn", "backend_unavailable") in codes(unavailable)
    wrong_launch = dataclasses.replace(
        fused, schedule=dataclasses.replace(fused.schedule, residual_norm_launch=NormLaunchParams(4, 4))
    )
    assert ("schedule.residual_norm_launch", "unsupported_launch_value") in codes(
        builder.evaluate(wrong_launch, small, _gfx950())
    )
    shadow = dataclasses.replace(
        fused,
        program=dataclasses.replace(
            fused.program,
            precision_plan=PrecisionPlan.FP16_FFN_INPUT_FP32_GELU,
            ffn_input_projection=ProjectionBackend.FP16_SHADOW,
        ),
    )
    assert ("program.ffn_input_projection", "backend_incompatible") in codes(builder.evaluate(shadow, small, _gfx950()))
    torch_norm = dataclasses.replace(
        fused,
        program=dataclasses.replace(fused.program, residual_norm=ResidualNormBackend.TORCH),
        schedule=dataclasses.replace(fused.schedule, residual_norm_launch=None),
    )
    assert ("program.residual_norm", "backend_incompatible") in codes(builder.evaluate(torch_norm, small, _gfx950()))
    # the reference's Triton fusion stays unavailable, not replaced
    triton = dataclasses.replace(
        fused, program=dataclasses.replace(fused.program, ffn=FFNBackend.TRITON_FUSED_MLP_BOUNDARY)
    )
    assert ("program.ffn", "backend_unavailable") in codes(builder.evaluate(triton, small, _gfx950()))


def test_narrow_widths_have_hip_norms():
    """The fused norm kernel covers 16-bit widths 128 and 256, so the gfx950
    program is legal at them."""

    builder = PlanBuilder()
    for width, heads in ((128, 2), (256, 4)):
        plan = builder.build(hip_config(), _context(batch=8, seq=128, d=width, heads=heads, ffn=4 * width), _gfx950())
        assert plan.use_hip_residual_norm


def test_linear_boundary_plans_and_rejections():
    """The HIP Linear + residual + LayerNorm boundary: accepted for 16-bit
    inference on gfx950 at widths 512 and 1024 with its launch, rejected with
    structured reasons otherwise (the reference's TRITON_LINEAR_MIXED rules,
    solution/plan_builder.py:668-707)."""

    import dataclasses

    from solution.config import (
        NormLaunchParams,
        PrecisionPlan,
        ProjectionBackend,
        ResidualNormBackend,
        RuntimeBackend,
        hip_linear_boundary_launch,
    )

    builder = PlanBuilder()
    codes = lambda result: {(v.field, v.code) for v in result.violations}  # noqa: E731
    fused = hip_config(residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED, boundary_launch=hip_linear_boundary_launch(512))
    assert fused.schedule.residual_norm_launch == NormLaunchParams(128, 8)
    assert fused.schedule.initial_norm_launch == NormLaunchParams(4, 4)
    assert ConfigSpec.from_dict(fused.to_dict()) == fused
    plan = builder.build(fused, _context(batch=64, seq=256, d=512, heads=8, ffn=2048, layers=4), _gfx950())
    assert plan.use_linear_boundary_fusion and plan.residual_norm_backend is ResidualNormBackend.HIP_LINEAR_FUSED
    assert plan.expected_trace.to_dict()["residual_norm_calls"] == 8
    long = hip_streamed_config(
        residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED, boundary_launch=hip_linear_boundary_launch(1024)
    )
    streamed = builder.build(long, _context(), _gfx950())
    assert streamed.use_streamed_execution and streamed.use_linear_boundary_fusion
    assert not builder.build(hip_config(), _context(), _gfx950()).use_linear_boundary_fusion
    with pytest.raises(ValueError, match="boundary_launch"):
        hip_config(residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED)
    with pytest.raises(ValueError, match="boundary_launch"):
        hip_config(boundary_launch=hip_linear_boundary_launch(1024))
    # the launch must be the width's: 1024-wide rows with the 512 launch
    wrong = builder.evaluate(fused, _context(), _gfx950())
    assert ("schedule.residual_norm_launch", "unsupported_launch_value") in codes(wrong)
    # widths without an instantiation (C4's 2048) are rejected, not replaced
    wide = hip_config(residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED, boundary_launch=NormLaunchParams(32, 8))
    rejected = builder.evaluate(wide, _context(batch=16, seq=4096, d=2048, heads=32, ffn=8192), _gfx950())
    assert ("program.residual_norm", "unsupported_shape") in codes(rejected)
    unavailable = builder.evaluate(long, _context(), _gfx950(hip_linear_residual_norm=False))
    assert ("program.residual_norm", "backend_unavailable") in codes(unavailable)
    fp32 = builder.evaluate(long, _context(dtype=torch.float32), _gfx950())
    assert ("program.residual_norm", "unsupported_dtype") in codes(fp32)
    masked = builder.evaluate(long, _context(mask=True), _gfx950())
    assert ("program.residual_norm", "mask_not_supported") in codes(masked)
    shadow = dataclasses.replace(
        long,
        program=dataclasses.replace(
            long.program,
            precision_plan=PrecisionPlan.FP16_FFN_OUTPUT,
            ffn_output_projection=ProjectionBackend.FP16_SHADOW,
        ),
    )
    assert ("program.ffn_output_projection", "backend_incompatible") in codes(builder.evaluate(shadow, _context(), _gfx950()))
    compiled = dataclasses.replace(
        fused,
        schedule=dataclasses.replace(fused.schedule, runtime=RuntimeBackend.COMPILED_FORWARD, compile_mode="max-autotune"),
    )
    c2 = _context(batch=64, seq=256, d=512, heads=8, ffn=2048, layers=4)
    assert ("schedule.runtime", "runtime_incompatible") in codes(builder.evaluate(compiled, c2, _gfx950()))
