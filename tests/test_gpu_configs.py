"""BASELINE.json's model configurations on the HIP path, at their own widths
and depths, through the programs the deployment registry publishes for them.

* C2 (B64 S256 D512 H8 F2048 L4) in full, and C4's workload (D2048 H32 F8192
  L2 at S=4096, one sequence of the B=16 batch) against the CPU oracle: the
  fp32 forward of the same rounded weights and inputs, and the official op
  order in bf16 (the reference path).  The gate is the model-level accuracy
  rule (autotune.accuracy, via oracle.compare.model_parity); the elementwise
  2e-2 / 1e-2 gate is printed beside it.
* C5's full sequence (S=100000, one sequence of the B=32 batch): every row of
  the streamed HIP program against the product's portable reference-order
  program (query-blocked torch attention, torch norms) run on the same GPU in
  bf16 and in fp32, which is how the reference checks its long-sequence
  program at measurement time (benchmarking/shape14_measure.py:139-162); the
  portable program itself is checked against the CPU oracle at small sizes
  (tests/test_operators_and_model.py).  The first 2048 rows are also
  checked against the CPU oracle (causality: they do not depend on later
  rows).
"""

from __future__ import annotations

import json
import os

import pytest
import torch

from oracle.compare import model_parity
from oracle.forward import TransformerConfig, cast_state, forward, generate_input, xavier_init_weights

pytestmark = pytest.mark.gpu


class _StateSource(torch.nn.Module):
    def __init__(self, tensors):
        super().__init__()
        self._tensors = tensors

    def state_dict(self, *args, **kwargs):
        return dict(self._tensors)


def _cpu_threads() -> None:
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))


def _deployed_program(d_model: int, seq_len: int):
    """The committed registry's program for the BASELINE shape of this width
    and length (whatever environment it was measured on)."""

    from deployment.registry import DEFAULT_DEPLOYED_CONFIGS_PATH
    from solution.config import ConfigSpec

    document = json.loads(DEFAULT_DEPLOYED_CONFIGS_PATH.read_text(encoding="utf-8"))
    for bundle in document["bundles"]:
        for entry in bundle["entries"]:
            shape = entry["shape"]
            if shape["qkv_dim"] == d_model and shape["seq_len"] == seq_len and shape["dtype"] == "bfloat16":
                return ConfigSpec.from_dict(entry["config"])
    raise AssertionError(f"no registry entry for D={d_model} S={seq_len}")


def _model(config, state, device, dtype, program):
    from solution.transformer import UserOptimizedTransformer, copy_model_weights

    model = UserOptimizedTransformer(config)
    copy_model_weights(_StateSource(state), model)
    model = model.to(device=device, dtype=dtype).eval()
    model.configure_execution(config=program)
    model.set_execution_observation(True)
    return model


def _oracle_pair(state, x, config, attention="auto"):
    """(fp32 forward of the bf16-rounded weights and input, bf16 official order)."""

    _cpu_threads()
    bf16_state = cast_state(state, torch.bfloat16)
    with torch.inference_mode():
        exact = forward(cast_state(bf16_state, torch.float32), x.float(), config, attention=attention)
        reference_path = forward(bf16_state, x, config, attention=attention).float()
    return exact, reference_path


def _assert_model(exact, reference_path, output, what):
    parity = model_parity(exact, reference_path, output.float().cpu())
    print(f"{what}: {parity.summary()}", flush=True)
    assert parity.passed, f"{what}: {parity.summary()}"


@pytest.mark.parametrize(
    "name,shape",
    [
        ("C2", (64, 256, 512, 8, 2048, 4)),
        ("C4 workload, one sequence", (1, 4096, 2048, 32, 8192, 2)),
    ],
)
def test_baseline_configuration_matches_the_oracle(gpu_device, name, shape):
    batch, seq, width, heads, ffn, layers = shape
    print(f"{name} {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=1234)
    x = generate_input(config, seed=1234).to(torch.bfloat16)
    program = _deployed_program(width, seq)
    model = _model(config, state, gpu_device, torch.bfloat16, program)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize(gpu_device)
    observed = model.describe_execution_path()["observed_execution_signature"]
    assert observed["attention_backend"] == "hip_streaming_dh64", observed
    del model
    exact, reference_path = _oracle_pair(state, x, config, attention="query_block" if seq > 1024 else "dense")
    _assert_model(exact, reference_path, output, f"{name} program {program.config_id[:16]}")


def test_long_sequence_every_row_matches_the_portable_program(gpu_device):
    from solution.config import portable_streamed_config
    from solution.shape14.defaults import hip_streamed_config

    seq, width, heads, ffn, layers = 100_000, 1024, 16, 4096, 2
    config = TransformerConfig(1, seq, width, heads, ffn, layers, True)
    print(f"C5 one sequence {config}", flush=True)
    state = xavier_init_weights(config, seed=1234)
    x = generate_input(config, seed=1234).to(torch.bfloat16)
    rounded = cast_state(state, torch.bfloat16)
    device_x = x.to(gpu_device)

    def run(program, dtype):
        model = _model(config, rounded, gpu_device, dtype, program)
        with torch.inference_mode():
            out = model(device_x.to(dtype))
        torch.cuda.synchronize(gpu_device)
        signature = model.describe_execution_path()["observed_execution_signature"]
        del model
        return out.float().cpu(), signature

    output, signature = run(hip_streamed_config(microbatch_size=1), torch.bfloat16)
    assert signature["attention_backend"] == "hip_streaming_dh64", signature
    reference_path, _ = run(portable_streamed_config(), torch.bfloat16)
    exact, reference_signature = run(portable_streamed_config(), torch.float32)
    assert reference_signature["attention_backend"] != "hip_streaming_dh64", reference_signature
    assert bool(torch.isfinite(output).all())
    _assert_model(exact, reference_path, output, "C5 S=100000 all rows vs portable program")
    # the late rows, whose 512-row blocks read the most keys
    late = slice(seq - 4096, seq)
    _assert_model(exact[:, late], reference_path[:, late], output[:, late], "C5 last 4096 rows")
    # the prefix against the CPU oracle: rows < 2048 see only keys < 2048
    prefix = TransformerConfig(1, 2048, width, heads, ffn, layers, True)
    exact_prefix, reference_prefix = _oracle_pair(state, x[:, :2048], prefix, attention="query_block")
    _assert_model(exact_prefix, reference_prefix, output[:, :2048], "C5 first 2048 rows vs CPU oracle")


def test_c1_fp32_configuration_on_the_hip_plan(gpu_device):
    """BASELINE C1 (B2 S128 D256 H4 F1024 L2, fp32, PyTorch default init,
    seed 1234) on the HIP plan for fp32 models (HIP fp32 attention, HIP fp32
    fused norms, fp32 hipBLASLt projections, torch's exact GELU) against the
    fp32 oracle and the committed float64 golden, at the fp32 gate
    |err| <= 1e-4 or |err| <= 1e-4 |ref|."""

    from pathlib import Path

    import numpy as np

    from oracle.compare import parity_gate
    from oracle.forward import default_init_weights
    from solution.config import FFNBackend, hip_config

    config = TransformerConfig(2, 128, 256, 4, 1024, 2, True)
    state = default_init_weights(config, seed=1234)
    x = generate_input(config, seed=1234)
    model = _model(config, state, gpu_device, torch.float32, hip_config(ffn=FFNBackend.TORCH))
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize(gpu_device)
    observed = model.describe_execution_path()["observed_execution_signature"]
    assert observed["attention_backend"] == "hip_streaming_dh64", observed
    assert observed["residual_norm_backend"] == "hip_fused", observed
    assert output.dtype == torch.float32
    _cpu_threads()
    with torch.inference_mode():
        reference = forward(state, x, config)
    golden = np.load(Path(__file__).resolve().parent / "golden" / "c1_forward.npz")
    for name, want in (("oracle fp32", reference), ("float64 golden", torch.from_numpy(golden["out"]))):
        result = parity_gate(want, output.cpu(), torch.float32)
        print(f"C1 vs {name}: max_abs={result.max_abs_error:.3g} failures={result.failed_elements}", flush=True)
        assert result.passed, f"C1 vs {name}: {result}"
