"""GPU parity of the gfx950 fused residual + LayerNorm/RMSNorm kernels.

Residuals are checked bitwise against the oracle (one rounding of the exact
sum to the stream dtype); normalized outputs use the parity gate written in
oracle.compare: 16-bit outputs pass elementwise with |err| <= 2e-2 or
|err| <= 1e-2 |ref|, fp32 outputs with 1e-4 / 1e-4.  The oracle computes the
statistics in float64 from the same rounded residual.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from oracle import norm as oracle_norm
from oracle.compare import parity_gate

pytestmark = pytest.mark.gpu


def _norm_module():
    from solution.kernels.norm import hip_residual

    return hip_residual


def _layer_norm(width, param_dtype, seed, device):
    generator = torch.Generator().manual_seed(seed)
    module = nn.LayerNorm(width)
    with torch.no_grad():
        module.weight.copy_(1 + 0.5 * torch.randn(width, generator=generator))
        module.bias.copy_(0.5 * torch.randn(width, generator=generator))
    return module.to(device=device, dtype=param_dtype)


def _assert_gate(reference, candidate, dtype, what):
    result = parity_gate(reference.float(), candidate.float().cpu(), dtype)
    assert result.passed, (
        f"{what}: {result.failed_elements}/{result.total_elements} failed, "
        f"max_abs={result.max_abs_error:.4g} at {result.worst_index}"
    )


@pytest.mark.parametrize(
    "value_dtype,update_dtype,normalized_dtype",
    [
        (torch.bfloat16, torch.bfloat16, torch.bfloat16),
        (torch.float16, torch.float16, torch.float16),
        (torch.float32, torch.float32, torch.float32),
        (torch.float32, torch.float16, torch.float16),
        (torch.float32, torch.float16, torch.float32),
        (torch.float32, torch.bfloat16, torch.bfloat16),
        (torch.float32, torch.bfloat16, torch.float32),
    ],
)
@pytest.mark.parametrize("width", [128, 256, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("rows", [1, 7, 1000])
def test_residual_layer_norm_matches_oracle(
    gpu_device, value_dtype, update_dtype, normalized_dtype, width, rows
):
    print(f"residual LN {value_dtype}/{update_dtype}/{normalized_dtype} {rows}x{width}", flush=True)
    module = _norm_module()
    generator = torch.Generator().manual_seed(rows * 31 + width)
    value = torch.randn(rows, width, generator=generator).to(value_dtype)
    update = torch.randn(rows, width, generator=generator).to(update_dtype)
    param_dtype = value_dtype
    layer_norm = _layer_norm(width, param_dtype, rows, gpu_device)
    with torch.inference_mode():
        residual, normalized, marker = module.hip_residual_layer_norm(
            value.to(gpu_device), update.to(gpu_device), layer_norm,
            normalized_dtype=normalized_dtype,
        )
    assert marker == module.HIP_RESIDUAL_LAYER_NORM_BACKEND
    ref_residual, ref_normalized = oracle_norm.residual_layer_norm(
        value, update, layer_norm.weight.detach().cpu(), layer_norm.bias.detach().cpu(),
        normalized_dtype=normalized_dtype,
    )
    assert residual.dtype == value_dtype and normalized.dtype == normalized_dtype
    assert torch.equal(residual.cpu(), ref_residual)
    _assert_gate(ref_normalized, normalized, normalized_dtype, "normalized")


@pytest.mark.parametrize("param_dtype", [torch.float32, torch.bfloat16])
def test_baseline_config3_norm(gpu_device, param_dtype):
    """BASELINE config 3's norm: [16384, 1024] bf16 N(0,1), gamma=1 beta=0 and
    random affine parameters."""

    module = _norm_module()
    generator = torch.Generator().manual_seed(1234)
    value = torch.randn(16384, 1024, generator=generator).to(torch.bfloat16)
    update = torch.randn(16384, 1024, generator=generator).to(torch.bfloat16)
    for layer_norm in (nn.LayerNorm(1024).to(gpu_device, param_dtype),
                       _layer_norm(1024, param_dtype, 7, gpu_device)):
        with torch.inference_mode():
            residual, normalized, _ = module.hip_residual_layer_norm(
                value.to(gpu_device), update.to(gpu_device), layer_norm
            )
        ref_residual, ref_normalized = oracle_norm.residual_layer_norm(
            value, update, layer_norm.weight.detach().cpu(), layer_norm.bias.detach().cpu()
        )
        assert torch.equal(residual.cpu(), ref_residual)
        _assert_gate(ref_normalized, normalized, torch.bfloat16, "config 3 norm")


def test_unit_affine_output_is_standardized(gpu_device):
    """gamma=1, beta=0: every row of the output has mean 0 and variance 1."""

    module = _norm_module()
    value = torch.randn(256, 1024, dtype=torch.float32) * 3 + 2
    update = torch.randn(256, 1024, dtype=torch.float32)
    layer_norm = nn.LayerNorm(1024).to(gpu_device)
    with torch.inference_mode():
        _, normalized, _ = module.hip_residual_layer_norm(
            value.to(gpu_device), update.to(gpu_device), layer_norm
        )
    normalized = normalized.double().cpu()
    assert normalized.mean(dim=-1).abs().max().item() < 1e-5
    assert (normalized.var(dim=-1, unbiased=False) - 1).abs().max().item() < 1e-3


def test_constant_rows_return_bias(gpu_device):
    module = _norm_module()
    value = torch.full((5, 512), 2.5, dtype=torch.bfloat16)
    update = torch.full((5, 512), -0.5, dtype=torch.bfloat16)
    layer_norm = _layer_norm(512, torch.bfloat16, 3, gpu_device)
    with torch.inference_mode():
        residual, normalized, _ = module.hip_residual_layer_norm(
            value.to(gpu_device), update.to(gpu_device), layer_norm
        )
    assert torch.all(residual.cpu() == 2.0)
    assert torch.equal(normalized.cpu(), layer_norm.bias.detach().cpu().expand(5, 512))


@pytest.mark.parametrize("width", [128, 256, 1024])
@pytest.mark.parametrize("block_rows,num_warps", [(1, 1), (2, 2), (4, 4), (8, 4), (16, 8), (64, 8)])
def test_launch_shapes_are_bitwise_identical(gpu_device, block_rows, num_warps, width):
    module = _norm_module()
    generator = torch.Generator().manual_seed(99)
    value = torch.randn(333, width, generator=generator).to(torch.bfloat16).to(gpu_device)
    update = torch.randn(333, width, generator=generator).to(torch.bfloat16).to(gpu_device)
    layer_norm = _layer_norm(width, torch.bfloat16, 1, gpu_device)
    with torch.inference_mode():
        base = module.hip_residual_layer_norm(value, update, layer_norm, block_rows=1, num_warps=1)
        other = module.hip_residual_layer_norm(
            value, update, layer_norm, block_rows=block_rows, num_warps=num_warps
        )
    assert torch.equal(base[0], other[0]) and torch.equal(base[1], other[1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rms_norm_matches_oracle(gpu_device, dtype):
    module = _norm_module()
    generator = torch.Generator().manual_seed(5)
    value = torch.randn(300, 2048, generator=generator).to(dtype)
    update = torch.randn(300, 2048, generator=generator).to(dtype)
    weight = (1 + 0.3 * torch.randn(2048, generator=generator)).to(dtype)
    with torch.inference_mode():
        residual, normalized, marker = module.hip_residual_rms_norm(
            value.to(gpu_device), update.to(gpu_device), weight.to(gpu_device), eps=1e-6
        )
        alone, _ = module.hip_rms_norm(residual, weight.to(gpu_device), eps=1e-6)
    assert marker == module.HIP_RESIDUAL_RMS_NORM_BACKEND
    ref_residual, ref_normalized = oracle_norm.residual_rms_norm(value, update, weight, 1e-6)
    assert torch.equal(residual.cpu(), ref_residual)
    _assert_gate(ref_normalized, normalized, dtype, "rms")
    assert torch.equal(alone, normalized)
    library_rms = torch.nn.functional.rms_norm(
        ref_residual.double(), (2048,), weight.double(), 1e-6
    )
    _assert_gate(library_rms, normalized, dtype, "rms vs torch.nn.functional.rms_norm")


@pytest.mark.parametrize(
    "value_dtype,normalized_dtype",
    [
        (torch.bfloat16, torch.bfloat16),
        (torch.float16, torch.float16),
        (torch.float32, torch.float32),
        (torch.float32, torch.float16),
        (torch.float32, torch.bfloat16),
    ],
)
@pytest.mark.parametrize("width", [128, 256, 1024])
def test_initial_layer_norm_matches_oracle(gpu_device, value_dtype, normalized_dtype, width):
    module = _norm_module()
    generator = torch.Generator().manual_seed(8)
    value = torch.randn(2, 513, width, generator=generator).to(value_dtype)
    layer_norm = _layer_norm(width, value_dtype, 2, gpu_device)
    with torch.inference_mode():
        normalized, marker = module.hip_layer_norm(
            value.to(gpu_device), layer_norm, normalized_dtype=normalized_dtype
        )
    assert marker == module.HIP_LAYER_NORM_BACKEND
    reference = oracle_norm.layer_norm(
        value, layer_norm.weight.detach().cpu(), layer_norm.bias.detach().cpu(),
        out_dtype=normalized_dtype,
    )
    _assert_gate(reference, normalized, normalized_dtype, "initial norm")


def test_output_can_be_a_slice_of_a_preallocated_buffer(gpu_device):
    """The streamed driver writes the final boundary straight into its output."""

    module = _norm_module()
    output = torch.zeros(4, 64, 1024, dtype=torch.bfloat16, device=gpu_device)
    value = torch.randn(2, 64, 1024).to(torch.bfloat16).to(gpu_device)
    update = torch.randn(2, 64, 1024).to(torch.bfloat16).to(gpu_device)
    layer_norm = _layer_norm(1024, torch.bfloat16, 4, gpu_device)
    with torch.inference_mode():
        _, normalized, _ = module.hip_residual_layer_norm(
            value, update, layer_norm, out=output[2:4]
        )
        _, expected, _ = module.hip_residual_layer_norm(value, update, layer_norm)
    assert normalized.data_ptr() == output[2:4].data_ptr()
    assert torch.equal(output[2:4], expected)
    assert torch.all(output[:2] == 0)


def test_ineligible_inputs_raise(gpu_device):
    module = _norm_module()
    value = torch.randn(4, 1000, device=gpu_device)  # width without an instantiation
    layer_norm = nn.LayerNorm(1000).to(gpu_device)
    with torch.inference_mode():
        with pytest.raises(RuntimeError, match="ineligible"):
            module.hip_residual_layer_norm(value, value, layer_norm)
        with pytest.raises(ValueError):
            module.hip_residual_layer_norm(value, value, layer_norm, block_rows=3, num_warps=2)
