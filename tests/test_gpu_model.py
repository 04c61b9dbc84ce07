"""GPU parity of the whole plugin model on the HIP plan.

"The reference PyTorch path on the same seeded inputs" is the oracle's
official-order forward in the model dtype (bf16 weights and activations,
fp32 softmax and statistics).  Two criteria, both from oracle.compare:

* fp32-output programs: the elementwise gate, |err| <= 2e-2 or
  |err| <= 1e-2 * |ref| for 16-bit internals.
* bf16-output programs (bf16 residual stream): model_parity -- compared with
  the fp32 forward of the same rounded weights and inputs, the HIP output must
  be no less accurate than the bf16 reference path (max-abs within 1.25x or
  2e-2, mean-abs within 1.25x, at most 1.25x as many elements outside the
  2e-2 / 1e-2 gate).  A strict elementwise gate between two bf16 pipelines is below the
  residual stream's noise floor (one ulp at |r| in [4, 8) is 0.03).
"""

from __future__ import annotations

import pytest
import torch

from oracle.compare import model_parity, parity_gate
from oracle.forward import TransformerConfig, cast_state, forward, generate_input, xavier_init_weights

pytestmark = pytest.mark.gpu


class _StateSource(torch.nn.Module):
    def __init__(self, tensors):
        super().__init__()
        self._tensors = tensors

    def state_dict(self, *args, **kwargs):
        return dict(self._tensors)


def _model(config, state, device, dtype):
    from solution.transformer import UserOptimizedTransformer, copy_model_weights

    model = UserOptimizedTransformer(config)
    copy_model_weights(_StateSource(state), model)
    return model.to(device=device, dtype=dtype).eval()


def _check(reference, output, dtype, what, fp32_reference=None):
    result = parity_gate(reference, output.float().cpu(), dtype)
    print(f"{what}: max_abs={result.max_abs_error:.4g} failed={result.failed_elements}", flush=True)
    assert result.passed, (
        f"{what}: {result.failed_elements}/{result.total_elements} failed, "
        f"max_abs={result.max_abs_error:.4g} at {result.worst_index}"
    )


def _check_bf16_model(exact, reference_path, output, what):
    parity = model_parity(exact, reference_path, output.float().cpu())
    print(f"{what}: {parity.summary()}", flush=True)
    assert parity.passed, f"{what}: {parity.summary()}"


@pytest.mark.parametrize(
    "shape",
    [
        (2, 256, 512, 8, 2048, 2),   # BASELINE config 2 widths, fewer sequences
        (1, 300, 1024, 16, 4096, 2),  # long-sequence widths, ragged length
        (2, 128, 2048, 32, 8192, 1),  # config 4 widths
    ],
)
def test_hip_plan_matches_the_bf16_reference_path(gpu_device, shape):
    from solution.config import hip_config

    batch, seq, width, heads, ffn, layers = shape
    print(f"model parity {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=1234)
    x = generate_input(config, seed=1234).to(torch.bfloat16)
    model = _model(config, state, gpu_device, torch.bfloat16)
    model.configure_execution(config=hip_config())
    model.set_execution_observation(True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize()
    reference = forward(cast_state(state, torch.bfloat16), x, config)
    exact = forward(cast_state(cast_state(state, torch.bfloat16), torch.float32), x.float(), config)
    _check_bf16_model(exact, reference.float(), output, f"hip model {shape}")
    description = model.describe_execution_path()
    observed = description["observed_execution_signature"]
    assert observed == description["expected_execution_signature"]
    assert observed["attention_backend"] == "hip_streaming_dh64"
    assert observed["residual_norm_backend"] == "hip_fused"
    assert observed["initial_norm_backend"] == "hip"


@pytest.mark.parametrize(
    "shape",
    [
        (2, 256, 512, 8, 2048, 2),   # BASELINE config 2 widths
        (1, 300, 1024, 16, 4096, 2),  # long-sequence widths, ragged length
        (2, 128, 2048, 32, 8192, 1),  # config 4 widths
    ],
)
@pytest.mark.parametrize("ffn_backend", ["hip_linear_exact_gelu", "hip_exact_gelu"])
def test_fused_ffn_input_plan_matches_the_bf16_reference_path(gpu_device, shape, ffn_backend):
    """The programs with a HIP FFN activation path (the fused Linear + bias +
    exact GELU, or hipBLASLt followed by the HIP elementwise GELU), end to end
    against the official bf16 path."""

    from solution.config import FFNBackend, hip_config

    batch, seq, width, heads, ffn, layers = shape
    print(f"{ffn_backend} model parity {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=4321)
    x = generate_input(config, seed=4321).to(torch.bfloat16)
    model = _model(config, state, gpu_device, torch.bfloat16)
    model.configure_execution(config=hip_config(ffn=FFNBackend(ffn_backend)))
    model.set_execution_observation(True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize()
    reference = forward(cast_state(state, torch.bfloat16), x, config)
    exact = forward(cast_state(cast_state(state, torch.bfloat16), torch.float32), x.float(), config)
    _check_bf16_model(exact, reference.float(), output, f"{ffn_backend} model {shape}")
    description = model.describe_execution_path()
    observed = description["observed_execution_signature"]
    assert observed == description["expected_execution_signature"]
    assert observed["ffn_backend"] == ffn_backend


@pytest.mark.parametrize(
    "shape",
    [
        (2, 256, 512, 8, 2048, 2),   # BASELINE config 2 widths
        (1, 300, 1024, 16, 4096, 2),  # long-sequence widths, ragged length
        (2, 128, 2048, 32, 8192, 1),  # config 4 widths
    ],
)
def test_native_qkv_plan_matches_the_bf16_reference_path(gpu_device, shape):
    """The program whose QKV projection writes head-major Q / K and the
    seq-contiguous V^T straight from its epilogue, end to end against the
    official bf16 path."""

    from solution.config import QKVMaterialization, hip_config

    batch, seq, width, heads, ffn, layers = shape
    print(f"native qkv model parity {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=2468)
    x = generate_input(config, seed=2468).to(torch.bfloat16)
    model = _model(config, state, gpu_device, torch.bfloat16)
    model.configure_execution(config=hip_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD))
    model.set_execution_observation(True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize()
    reference = forward(cast_state(state, torch.bfloat16), x, config)
    exact = forward(cast_state(cast_state(state, torch.bfloat16), torch.float32), x.float(), config)
    _check_bf16_model(exact, reference.float(), output, f"native qkv model {shape}")
    description = model.describe_execution_path()
    observed = description["observed_execution_signature"]
    assert observed == description["expected_execution_signature"]
    assert observed["qkv_materialization"] == "hip_native_bhsd"


@pytest.mark.parametrize(
    "shape",
    [
        (2, 256, 512, 8, 2048, 2),   # BASELINE config 2 widths
        (1, 300, 1024, 16, 4096, 2),  # long-sequence widths, ragged length
    ],
)
def test_linear_boundary_plan_matches_the_bf16_reference_path(gpu_device, shape):
    """The program whose output projections are fused into their residual
    LayerNorm boundaries, end to end against the official bf16 path."""

    from solution.config import ResidualNormBackend, hip_config, hip_linear_boundary_launch

    batch, seq, width, heads, ffn, layers = shape
    print(f"linear boundary model parity {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=1357)
    x = generate_input(config, seed=1357).to(torch.bfloat16)
    model = _model(config, state, gpu_device, torch.bfloat16)
    model.configure_execution(
        config=hip_config(
            residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED, boundary_launch=hip_linear_boundary_launch(width)
        )
    )
    model.set_execution_observation(True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize()
    reference = forward(cast_state(state, torch.bfloat16), x, config)
    exact = forward(cast_state(cast_state(state, torch.bfloat16), torch.float32), x.float(), config)
    _check_bf16_model(exact, reference.float(), output, f"linear boundary model {shape}")
    description = model.describe_execution_path()
    observed = description["observed_execution_signature"]
    assert observed == description["expected_execution_signature"]
    assert observed["residual_norm_backend"] == "hip_linear_fused"


@pytest.mark.parametrize("program", ["default", "all_fused"])
@pytest.mark.parametrize("shape", [(2, 256, 512, 8, 2048, 2), (1, 300, 1024, 16, 4096, 1)])
def test_hip_programs_on_an_fp16_model_match_the_fp16_reference_path(gpu_device, shape, program):
    """Every HIP kernel also takes fp16 operands: the gfx950 program on an
    fp16 model (the default program, and the one with every fused GEMM
    epilogue), end to end against the official path run in fp16."""

    from solution.config import (
        FFNBackend,
        QKVMaterialization,
        ResidualNormBackend,
        hip_config,
        hip_linear_boundary_launch,
    )

    batch, seq, width, heads, ffn, layers = shape
    print(f"fp16 model parity {program} {shape}", flush=True)
    options = {}
    if program == "all_fused":
        options = dict(
            ffn=FFNBackend.HIP_LINEAR_EXACT_GELU,
            qkv=QKVMaterialization.HIP_NATIVE_BHSD,
            residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED,
            boundary_launch=hip_linear_boundary_launch(width),
        )
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=97)
    x = generate_input(config, seed=97).to(torch.float16)
    model = _model(config, state, gpu_device, torch.float16)
    model.configure_execution(config=hip_config(**options))
    model.set_execution_observation(True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize()
    assert output.dtype == torch.float16
    reference = forward(cast_state(state, torch.float16), x, config)
    exact = forward(cast_state(cast_state(state, torch.float16), torch.float32), x.float(), config)
    _check_bf16_model(exact, reference.float(), output, f"fp16 {program} model {shape}")
    description = model.describe_execution_path()
    observed = description["observed_execution_signature"]
    assert observed == description["expected_execution_signature"]
    assert observed["attention_compute_dtype"] == "float16"


def test_graph_runtime_replays_the_fused_projection_programs(gpu_device):
    """The graph-replay runtime with every fused GEMM epilogue and prologue
    (the initial LayerNorm fused into the native-layout QKV projection,
    Linear + exact GELU, the Linear + residual + LayerNorm boundaries):
    several replays with new inputs, eager work
    and synchronizations between them, each bitwise equal to the eager
    program on the same input."""

    from solution.config import (
        FFNBackend,
        InitialNormBackend,
        QKVMaterialization,
        ResidualNormBackend,
        hip_config,
        hip_linear_boundary_launch,
    )

    config = TransformerConfig(4, 256, 512, 8, 2048, 2, True)
    state = xavier_init_weights(config, seed=13)
    options = dict(
        ffn=FFNBackend.HIP_LINEAR_EXACT_GELU,
        qkv=QKVMaterialization.HIP_NATIVE_BHSD,
        residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED,
        boundary_launch=hip_linear_boundary_launch(512),
        initial_norm=InitialNormBackend.HIP_FUSED_QKV,
    )
    graph_model = _model(config, state, gpu_device, torch.bfloat16)
    graph_model.configure_execution(config=hip_config(graph=True, **options))
    eager_model = _model(config, state, gpu_device, torch.bfloat16)
    eager_model.configure_execution(config=hip_config(**options))
    with torch.inference_mode():
        for seed in (1, 2, 3):
            print(f"fused graph replay input seed {seed}", flush=True)
            x = generate_input(config, seed=seed).to(torch.bfloat16).to(gpu_device)
            replayed = graph_model(x)
            torch.cuda.synchronize()
            expected = eager_model(x)
            torch.cuda.synchronize()
            assert torch.equal(replayed, expected), f"replay {seed} differs from eager"


@pytest.mark.parametrize("boundary", ["hip_fused", "hip_linear_fused"])
def test_streamed_output_equals_its_chunks_bitwise(gpu_device, boundary):
    """The streamed driver runs ordered chunks and writes each chunk's final
    norm into the logical output: identical to running the chunks alone
    (with the residual-norm boundaries, or with the fused linear boundary
    writing the last chunk's output in place)."""

    from solution.config import ResidualNormBackend, hip_config, hip_linear_boundary_launch

    options = {}
    if boundary == "hip_linear_fused":
        options = dict(residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED, boundary_launch=hip_linear_boundary_launch(512))
    config = TransformerConfig(4, 200, 512, 8, 2048, 2, True)
    state = xavier_init_weights(config, seed=7)
    x = generate_input(config, seed=7).to(torch.bfloat16).to(gpu_device)
    streamed = _model(config, state, gpu_device, torch.bfloat16)
    streamed.configure_execution(config=hip_config(microbatch_size=2, **options))
    eager = _model(TransformerConfig(2, 200, 512, 8, 2048, 2, True), state, gpu_device, torch.bfloat16)
    eager.configure_execution(config=hip_config(**options))
    with torch.inference_mode():
        whole = streamed(x)
        parts = torch.cat([eager(x[0:2]), eager(x[2:4])])
    assert torch.equal(whole, parts)
    assert streamed.describe_execution_path()["runtime_backend"] == "streamed"


def test_long_sequence_forward_prefix_matches_the_oracle(gpu_device):
    """A 100 000-token forward at the long-sequence configuration's widths
    (D1024 H16 F4096 L2, bf16).  Causality makes its first rows a function of
    the prefix only, so they are checked against the oracle on that prefix."""

    from solution.shape14.defaults import hip_streamed_config

    seq, prefix = 100_000, 1024
    config = TransformerConfig(1, seq, 1024, 16, 4096, 2, True)
    state = xavier_init_weights(config, seed=2024)
    x = generate_input(config, seed=2024).to(torch.bfloat16)
    model = _model(config, state, gpu_device, torch.bfloat16)
    model.configure_execution(config=hip_streamed_config(microbatch_size=1))
    print("long-sequence forward S=100000", flush=True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize()
    assert torch.isfinite(output).all()
    prefix_config = TransformerConfig(1, prefix, 1024, 16, 4096, 2, True)
    reference = forward(cast_state(state, torch.bfloat16), x[:, :prefix], prefix_config)
    exact = forward(cast_state(cast_state(state, torch.bfloat16), torch.float32), x[:, :prefix].float(), prefix_config)
    _check_bf16_model(exact, reference.float(), output[:, :prefix], "S=100000 prefix rows")


def test_reference_shape14_program_with_hip_kernels_on_an_fp32_model(gpu_device):
    """The reference's deployed mixed-precision program (fp32 I/O, FP16 shadow
    projections) with the attention and norms swapped to the HIP kernels."""

    from solution.config import (
        AttentionLaunchParams,
        ConfigSpec,
        NormLaunchParams,
        ProgramConfig,
        RuntimeBackend,
        ScheduleConfig,
    )

    config = TransformerConfig(2, 256, 512, 8, 2048, 2, True)
    state = xavier_init_weights(config, seed=3)
    x = generate_input(config, seed=3)
    program = ProgramConfig(
        attention="hip_streaming_dh64",
        qkv_projection="fp16_shadow",
        attention_output_projection="fp16_shadow",
        ffn_input_projection="fp16_shadow",
        ffn_output_projection="fp16_shadow",
        precision_plan="fp16_core",
        qkv_materialization="view",
        attention_output_bridge="attention_direct_bsd",
        ffn="torch",
        residual_norm="hip_mixed",
        initial_norm="hip",
    )
    schedule = ScheduleConfig(
        runtime=RuntimeBackend.EAGER,
        attention_launch=AttentionLaunchParams(128, 64, 4, 2),
        residual_norm_launch=NormLaunchParams(4, 4),
        initial_norm_launch=NormLaunchParams(4, 4),
    )
    model = _model(config, state, gpu_device, torch.float32)
    model.configure_execution(config=ConfigSpec(program=program, schedule=schedule))
    model.set_execution_observation(True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    assert output.dtype == torch.float32
    reference = forward(state, x, config)
    _check(reference, output, torch.float16, "mixed fp16 program")
    observed = model.describe_execution_path()["observed_execution_signature"]
    assert observed["residual_norm_backend"] == "hip_mixed" and observed["complete"]


def test_graph_runtime_replays_equal_eager_execution(gpu_device):
    """The graph-replay runtime (a HIP graph per input signature) on the
    short-sequence configuration's widths: several replays with new inputs,
    eager work and synchronizations between them, each bitwise equal to the
    eager program on the same input."""

    from solution.config import hip_config

    config = TransformerConfig(8, 256, 512, 8, 2048, 2, True)
    state = xavier_init_weights(config, seed=11)
    graph_model = _model(config, state, gpu_device, torch.bfloat16)
    graph_model.configure_execution(config=hip_config(graph=True))
    graph_model.set_execution_observation(True)
    eager_model = _model(config, state, gpu_device, torch.bfloat16)
    eager_model.configure_execution(config=hip_config())
    with torch.inference_mode():
        for seed in (1, 2, 3, 4):
            print(f"graph replay input seed {seed}", flush=True)
            x = generate_input(config, seed=seed).to(torch.bfloat16).to(gpu_device)
            replayed = graph_model(x)
            torch.cuda.synchronize()
            expected = eager_model(x)
            torch.cuda.synchronize()
            assert torch.equal(replayed, expected), f"replay {seed} differs from eager"
        observed = graph_model.describe_execution_path()
        assert observed["runtime_backend"] == "cuda_graph"
        with pytest.raises(RuntimeError, match="one static input signature"):
            graph_model(torch.zeros(4, 256, 512, dtype=torch.bfloat16, device=gpu_device))


def test_default_resolution_on_gfx950_selects_the_hip_program(gpu_device):
    from solution.config import hip_config

    config = TransformerConfig(2, 64, 512, 8, 1024, 1, True)
    model = _model(config, xavier_init_weights(config, seed=1), gpu_device, torch.bfloat16)
    x = generate_input(config, seed=1).to(torch.bfloat16).to(gpu_device)
    with torch.inference_mode():
        model(x)
    assert model.describe_execution_path()["planned_config_id"] == hip_config().config_id


def test_default_resolution_selects_the_published_registry_entry(gpu_device):
    """A shape published in the deployment registry for this environment runs
    the published program without configure_execution (the reference's
    exact-match resolution, deployment/registry.py)."""

    from deployment.environment import EnvironmentFingerprint, ImplementationScope
    from deployment.registry import ShapeFingerprint, resolve_deployed_config

    import json

    from deployment.registry import DEFAULT_DEPLOYED_CONFIGS_PATH

    config = TransformerConfig(64, 256, 512, 8, 2048, 4, True)
    detected = EnvironmentFingerprint.detect(gpu_device, scope=ImplementationScope.RESIDENT)
    published = resolve_deployed_config(
        hardware=detected,
        shape=ShapeFingerprint(
            batch_size=64, qkv_dim=512, heads=8, seq_len=256, layers=4, causal=True, ffn_dim=2048,
            dtype="bfloat16", padding_ratio=0.0, input_scale=1.0,
        ),
    )
    if published is None:
        # name the fields that keep every committed bundle from matching
        document = json.loads(DEFAULT_DEPLOYED_CONFIGS_PATH.read_text(encoding="utf-8"))
        mine = detected.to_dict()
        for bundle in document["bundles"]:
            theirs = bundle["hardware"]
            differing = {
                key: (theirs.get(key), mine[key])
                for key in mine
                if key not in ("official_definitions_digest", "solution_implementation_digest")
                and theirs.get(key) != mine[key]
            }
            print(f"bundle {theirs.get('scope')}: fields differing (committed, detected): {differing}", flush=True)
    assert published is not None, "the committed registry holds no entry for this environment's fingerprint"
    model = _model(config, xavier_init_weights(config, seed=3), gpu_device, torch.bfloat16)
    x = generate_input(config, seed=3).to(torch.bfloat16).to(gpu_device)
    with torch.inference_mode():
        model(x)
    assert model.describe_execution_path()["planned_config_id"] == published.config_id
