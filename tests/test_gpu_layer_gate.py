"""The north-star elementwise gate on each layer of the models, and the
official harness's call form, on the HIP plan.

* Per layer, teacher-forced: each HIP layer is fed the reference path's own
  bf16 input for that layer (the official op order in bf16, computed by the
  oracle).  Three comparisons per layer:
  - the attention sub-layer: the HIP kernel on the reference path's own q,
    k, v (real activations at the configuration's full shape) against the
    fp32 attention of the same bf16 q, k, v, at the gate |err| <= 2e-2 or
    |err| <= 1e-2 |ref|, every element (the bf16 official order, which
    rounds the scores and P to bf16, is printed beside it);
  - the first residual boundary: the HIP fused residual + LayerNorm on the
    reference path's own residual and attention update: the residual equal
    bit for bit (one fp32 add, one rounding, as torch), the normalized output
    at the gate, every element;
  - the whole layer (the next LayerNorm of the layer's residual, what the
    following layer or the model output consumes) against the reference
    path's.  Two bf16 pipelines that round at different points differ here
    by 2-3 ulps of bf16 (0.031-0.047 on values of magnitude 2-3) in 1e-4 to
    3e-4 of the elements, and the reference path itself misses the gate
    against the fp32 layer in as many elements as the HIP layer does, so the
    strict gate is not attainable for any bf16 layer that rounds differently
    from the reference path.  The layer is held to at most 1e-3 of its
    elements outside the strict gate against the reference path, and,
    against the fp32 layer, to no more elements outside the gate and no
    larger max-abs error than the reference path (x1.25, the model-level
    spread).
  C2 (B64 S256 D512 H8 F2048 L4) and C4's workload (one sequence, S4096
  D2048 H32 F8192 L2) with the registry programs, the reference path on the
  CPU; C5's widths at S=100000 (one sequence, D1024 H16 F4096 L2) with the
  long-sequence program, the reference path run by the oracle on the GPU.
* The harness call form: official/torch_transformer_benchmark.py builds an
  all-True mask (:256-259) and calls model(x, valid_mask) (:472,494,504); the
  model collapses it so the mask-free HIP kernels stay legal
  (solution/transformer.py:1646-1675).  The output must equal the mask-free
  call's bit for bit and the observed execution must be the HIP one.
* fp32 I/O with fp16 internals at C5's widths (B=1, S=100000): the check the
  reference runs before timing its long-sequence shape
  (benchmarking/shape14_measure.py:139-162) on the program closest to its
  deployed one -- fp32 residual stream, fp16 projections and attention -- with
  the HIP attention and mixed norms, against the fp32 portable program under
  the official rule (rtol 0.02, atol 0.002, ratio <= 1 passes), at C5's
  widths and on the reference's own Shape 14 (F=1024, PyTorch default init),
  where the reference recorded 0.2816 with its Triton program.
"""

from __future__ import annotations

import json
import math
import os

import pytest
import torch
import torch.nn.functional as F

from oracle.compare import OFFICIAL_ATOL, OFFICIAL_RTOL, official_compare, parity_gate
from oracle.forward import (
    TransformerConfig,
    attention_inputs,
    cast_state,
    dense_causal_attention,
    final_norm,
    generate_input,
    layer_output,
    query_block_causal_attention,
    xavier_init_weights,
)

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


def _single_layer_state(state, index: int, layers: int):
    """Layer ``index`` as a one-layer model whose final LayerNorm is the norm
    that follows the layer in the full model (the next layer's norm1, or the
    final norm after the last layer)."""

    prefix = f"layers.{index}."
    single = {"layers.0." + name[len(prefix):]: tensor for name, tensor in state.items() if name.startswith(prefix)}
    following = f"layers.{index + 1}.norm1" if index + 1 < layers else "final_norm"
    single["final_norm.weight"] = state[following + ".weight"]
    single["final_norm.bias"] = state[following + ".bias"]
    return single


def _reference_layer(single, x, heads, attention):
    """One layer in the official op order, in the dtype of ``x`` and ``single``:
    (the layer's residual output, the following LayerNorm of it)."""

    scale = (x.shape[-1] // heads) ** -0.5
    q, k, v = attention_inputs(single, x, 0, heads)
    residual = layer_output(single, x, attention(q, k, v, scale), 0)
    return residual, final_norm(single, residual)


def _sublayers(name, index, single, x, heads, attention, program, device):
    """The HIP attention on the reference path's own q, k, v, and the HIP
    residual LayerNorm on its own residual and attention update."""

    from solution.kernels.norm.hip_residual import hip_residual_layer_norm
    from solution.shape14.hip_streaming_dh64 import hip_streaming_dh64_causal_attention_bsd

    batch, seq, width = x.shape
    scale = (width // heads) ** -0.5
    launch = program.schedule.attention_launch
    q, k, v = attention_inputs(single, x, 0, heads)
    context = attention(q, k, v, scale).transpose(1, 2).reshape(batch, seq, width)
    exact_context = attention(q.float(), k.float(), v.float(), scale).transpose(1, 2).reshape(batch, seq, width)
    hip_context, _ = hip_streaming_dh64_causal_attention_bsd(
        q.to(device), k.to(device), v.to(device), scale=scale, block_m=launch.block_m,
        num_warps=launch.num_warps, num_stages=launch.num_stages,
    )
    torch.cuda.synchronize(device)
    # The kernel against the fp32 attention of the same bf16 q, k, v (the
    # kernel's own contract); the bf16 official order beside it, which
    # rounds the scores and P to bf16 on the way.
    exact_context = exact_context.cpu()
    attention_gate = parity_gate(exact_context, hip_context.float().cpu(), torch.bfloat16)
    official_gate = parity_gate(exact_context, context.float().cpu(), torch.bfloat16)
    print(f"{name} layer {index} attention on the reference q, k, v, against fp32: HIP "
          f"max_abs={attention_gate.max_abs_error:.4g} failed={attention_gate.failed_elements}/"
          f"{attention_gate.total_elements}; bf16 official order max_abs={official_gate.max_abs_error:.4g} "
          f"failed={official_gate.failed_elements}", flush=True)
    del exact_context
    update = F.linear(context, single["layers.0.attention.out_proj.weight"], single["layers.0.attention.out_proj.bias"])
    residual = x + update
    normalized = F.layer_norm(residual, (width,), single["layers.0.norm2.weight"], single["layers.0.norm2.bias"], 1e-5)
    norm = torch.nn.LayerNorm(width, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(single["layers.0.norm2.weight"])
        norm.bias.copy_(single["layers.0.norm2.bias"])
    launch = program.schedule.residual_norm_launch
    hip_residual, hip_normalized, _ = hip_residual_layer_norm(
        x.to(device), update.to(device), norm, block_rows=launch.block_rows, num_warps=launch.num_warps
    )
    torch.cuda.synchronize(device)
    norm_gate = parity_gate(normalized.float().cpu(), hip_normalized.float().cpu(), torch.bfloat16)
    residual_equal = torch.equal(hip_residual.cpu(), residual.cpu())
    print(f"{name} layer {index} residual LayerNorm on the reference residual and update: residual bitwise "
          f"{residual_equal}, normalized max_abs={norm_gate.max_abs_error:.4g} "
          f"failed={norm_gate.failed_elements}", flush=True)
    return attention_gate, residual_equal, norm_gate


def _teacher_forced(name, shape, program, device, reference_device):
    batch, seq, width, heads, ffn, layers = shape
    attention = query_block_causal_attention if seq > 1024 else dense_causal_attention
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=1234)
    bf16_state = cast_state(state, torch.bfloat16)
    single_config = TransformerConfig(batch, seq, width, heads, ffn, 1, True)
    x = generate_input(config, seed=1234).to(torch.bfloat16).to(reference_device)
    _cpu_threads()
    problems = []
    for index in range(layers):
        single = _single_layer_state(bf16_state, index, layers)
        print(f"{name} layer {index}: reference path", flush=True)
        with torch.inference_mode():
            ref_single = {key: tensor.to(reference_device) for key, tensor in single.items()}
            attention_gate, residual_equal, norm_gate = _sublayers(
                name, index, ref_single, x, heads, attention, program, device
            )
            next_x, expected = _reference_layer(ref_single, x, heads, attention)
            fp32_single = cast_state(ref_single, torch.float32)
            _, exact = _reference_layer(fp32_single, x.float(), heads, attention)
        model = _model(single_config, single, device, torch.bfloat16, program)
        with torch.inference_mode():
            output = model(x.to(device))
        torch.cuda.synchronize(device)
        observed = model.describe_execution_path()["observed_execution_signature"]
        assert observed["attention_backend"] == "hip_streaming_dh64", observed
        del model
        candidate = output.float().cpu()
        expected, exact = expected.float().cpu(), exact.float().cpu()
        gate = parity_gate(expected, candidate, torch.bfloat16)
        reference_vs_fp32 = parity_gate(exact, expected, torch.bfloat16)
        candidate_vs_fp32 = parity_gate(exact, candidate, torch.bfloat16)
        print(
            f"{name} layer {index}: vs reference path max_abs={gate.max_abs_error:.4g} "
            f"strict-gate failures={gate.failed_elements}/{gate.total_elements}; vs fp32: candidate "
            f"max_abs={candidate_vs_fp32.max_abs_error:.4g} failed={candidate_vs_fp32.failed_elements}, "
            f"reference path max_abs={reference_vs_fp32.max_abs_error:.4g} "
            f"failed={reference_vs_fp32.failed_elements}",
            flush=True,
        )
        if not attention_gate.passed:
            problems.append(f"layer {index}: attention sub-layer {attention_gate}")
        if not residual_equal:
            problems.append(f"layer {index}: the HIP residual differs from the reference add")
        if not norm_gate.passed:
            problems.append(f"layer {index}: residual LayerNorm sub-layer {norm_gate}")
        if gate.failed_elements > 1e-3 * gate.total_elements:
            problems.append(f"layer {index}: {gate.failed_elements} elements outside the strict gate")
        if candidate_vs_fp32.failed_elements > 1.25 * reference_vs_fp32.failed_elements + 1e-5 * gate.total_elements:
            problems.append(f"layer {index}: more elements outside the gate against fp32 than the reference path")
        if candidate_vs_fp32.max_abs_error > max(2e-2, 1.25 * reference_vs_fp32.max_abs_error):
            problems.append(f"layer {index}: larger error against fp32 than the reference path")
        x = next_x
        del output, candidate, expected, exact
    assert not problems, f"{name}: " + "; ".join(problems)


@pytest.mark.parametrize(
    "name,shape",
    [
        ("C2", (64, 256, 512, 8, 2048, 4)),
        ("C4 workload, one sequence", (1, 4096, 2048, 32, 8192, 2)),
    ],
)
def test_each_layer_meets_the_elementwise_gate(gpu_device, name, shape):
    program = _deployed_program(shape[2], shape[1])
    _teacher_forced(name, shape, program, gpu_device, torch.device("cpu"))


def test_each_long_sequence_layer_meets_the_elementwise_gate(gpu_device):
    from solution.shape14.defaults import hip_streamed_config

    _teacher_forced(
        "C5 widths, S=100000",
        (1, 100_000, 1024, 16, 4096, 2),
        hip_streamed_config(microbatch_size=1),
        gpu_device,
        gpu_device,
    )


@pytest.mark.parametrize(
    "name,shape,inference_mask",
    [
        ("C2", (64, 256, 512, 8, 2048, 4), False),
        ("C2, mask made under inference_mode", (64, 256, 512, 8, 2048, 4), True),
        ("C5 widths, one sequence", (1, 100_000, 1024, 16, 4096, 2), False),
    ],
)
def test_harness_call_form_with_an_all_true_mask(gpu_device, name, shape, inference_mask):
    from solution.shape14.defaults import hip_streamed_config

    batch, seq, width, heads, ffn, layers = shape
    print(f"harness call form {name} {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=77)
    program = hip_streamed_config(microbatch_size=1) if seq > 4096 else _deployed_program(width, seq)
    model = _model(config, state, gpu_device, torch.bfloat16, program)
    x = generate_input(config, seed=77, dtype=torch.bfloat16, device=gpu_device)
    if inference_mask:
        with torch.inference_mode():
            valid_mask = torch.ones(batch, seq, device=gpu_device, dtype=torch.bool)
    else:
        valid_mask = torch.ones(batch, seq, device=gpu_device, dtype=torch.bool)
    with torch.inference_mode():
        masked = model(x, valid_mask)
        torch.cuda.synchronize(gpu_device)
        description = model.describe_execution_path()
        observed = description["observed_execution_signature"]
        expected = description["expected_execution_signature"]
        # the same tensor again (the reference caches its classification)
        again = model(x, valid_mask)
        unmasked = model(x)
    torch.cuda.synchronize(gpu_device)
    assert observed["attention_backend"] == "hip_streaming_dh64", observed
    assert observed["residual_norm_backend"] == "hip_fused", observed
    assert observed["initial_norm_backend"] == "hip", observed
    assert observed["complete"], observed
    for field in ("attention_backend", "residual_norm_backend", "initial_norm_backend", "ffn_backend"):
        assert observed[field] == expected[field], (field, observed, expected)
    assert torch.equal(masked, unmasked), f"{name}: masked call differs from the mask-free call"
    assert torch.equal(again, unmasked)


@pytest.mark.parametrize(
    "program_name,ffn,init",
    [
        # BASELINE C5's widths (F=4096) with its Xavier-uniform weights
        ("hip_deployed_shape14_config", 4096, "xavier"),
        ("hip_mixed_streamed_config", 4096, "xavier"),
        # the reference's own Shape 14 (F=1024, PyTorch default init), the
        # configuration its recorded ratio of 0.2816 was measured on
        ("hip_deployed_shape14_config", 1024, "default"),
    ],
)
def test_fp32_io_long_sequence_meets_the_official_rule(gpu_device, program_name, ffn, init):
    from autotune.accuracy import gate_ratio
    from oracle.forward import default_init_weights
    from solution.config import portable_streamed_config
    from solution.shape14 import defaults

    seq, width, heads, layers = 100_000, 1024, 16, 2
    config = TransformerConfig(1, seq, width, heads, ffn, layers, True)
    print(f"fp32 I/O {program_name} {init} init {config}", flush=True)
    state = (xavier_init_weights if init == "xavier" else default_init_weights)(config, seed=1234)
    x = generate_input(config, seed=1234, device=gpu_device)

    def run(program):
        model = _model(config, state, gpu_device, torch.float32, program)
        with torch.inference_mode():
            out = model(x)
        torch.cuda.synchronize(gpu_device)
        signature = model.describe_execution_path()["observed_execution_signature"]
        del model
        return out, signature

    candidate, signature = run(getattr(defaults, program_name)(microbatch_size=1))
    assert candidate.dtype == torch.float32
    assert signature["attention_backend"] == "hip_streaming_dh64", signature
    assert signature["attention_compute_dtype"] == "float16", signature
    assert signature["residual_norm_backend"] in {"hip_fused", "hip_mixed"}, signature
    reference, reference_signature = run(portable_streamed_config())
    assert reference_signature["attention_backend"] != "hip_streaming_dh64", reference_signature
    ratio = gate_ratio(candidate, reference, atol=OFFICIAL_ATOL, rtol=OFFICIAL_RTOL)
    comparison = official_compare(reference, candidate, rtol=OFFICIAL_RTOL, atol=OFFICIAL_ATOL)
    print(
        f"fp32 I/O {program_name} F={ffn} {init} init S=100000: official ratio {ratio:.4f} "
        f"(reference's recorded 0.2816 at F=1024, default init), max_abs={comparison.max_abs_error:.4g} "
        f"failed={comparison.failed_elements}/{comparison.total_elements}",
        flush=True,
    )
    assert math.isfinite(ratio)
    assert comparison.passed and ratio <= 1.0
