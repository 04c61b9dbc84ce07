"""GPU parity of the initial LayerNorm fused into the QKV projection
(sah_norm_qkv_projection, the HIP_FUSED_QKV initial norm).

Three references:

* the unfused HIP pair on the same operands, ``sah_norm`` (LayerNorm into a
  16-bit buffer) then ``sah_qkv_projection``: the fused kernel forms the row
  statistics exactly as the norm kernel does and rounds the normalized row
  to the operand dtype before its MFMAs, so Q / K / V must be equal bit for
  bit.  A statistic formed another way, a weight or bias chunk applied to
  the wrong columns, or a missing rounding breaks equality.
* float64 on the CPU: ``F.layer_norm`` in float64 from the same 16-bit x,
  weight and bias, rounded to the operand dtype (the model's boundary
  rounding), then ``F.linear`` with the packed weight in float64.  Every
  element must pass the 16-bit gate and lie within a few output ulps; a
  dropped mean, a wrong variance divisor or eps, or unnormalized input fails
  by far.
* the whole model: the fused program's output equals the unfused program's
  bit for bit, and passes the model-level accuracy rule against the CPU
  oracle.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle.compare import model_parity, parity_gate
from oracle.forward import TransformerConfig, cast_state, forward, generate_input, xavier_init_weights

pytestmark = pytest.mark.gpu


def _operands(batch, seq, d_model, dtype, seed, device):
    g = torch.Generator().manual_seed(seed)
    # rows with their own offsets and spreads, so the statistics matter
    x = 3.0 * torch.randn(batch, seq, 1, generator=g) + (0.5 + 2.0 * torch.rand(batch, seq, 1, generator=g)) * torch.randn(
        batch, seq, d_model, generator=g
    )
    w = (torch.rand(3 * d_model, d_model, generator=g) * 2 - 1) * (6.0 / (4 * d_model)) ** 0.5
    b = 0.2 * torch.randn(3 * d_model, generator=g)
    ln_w = 1.0 + 0.3 * torch.randn(d_model, generator=g)
    ln_b = 0.2 * torch.randn(d_model, generator=g)
    host = tuple(t.to(dtype) for t in (x, w, b, ln_w, ln_b))
    return host, tuple(t.to(device) for t in host)


def _layer_norm(weight, bias, device):
    norm = torch.nn.LayerNorm(weight.numel(), device=device, dtype=weight.dtype)
    with torch.no_grad():
        norm.weight.copy_(weight)
        norm.bias.copy_(bias)
    return norm


def _float64_reference(x, w, b, ln_w, ln_b, heads, eps):
    batch, seq, d_model = x.shape
    y = F.layer_norm(x.double(), (d_model,), ln_w.double(), ln_b.double(), eps).to(x.dtype)
    packed = F.linear(y.double(), w.double(), b.double())
    parts = packed.split(d_model, dim=-1)
    return tuple(p.reshape(batch, seq, heads, d_model // heads).transpose(1, 2) for p in parts)


@pytest.mark.parametrize(
    "batch,seq,d_model,heads,dtype",
    [
        (2, 256, 512, 8, torch.bfloat16),     # C2 widths
        (3, 77, 512, 8, torch.bfloat16),      # rows not a multiple of the tile, ragged sequences
        (1, 300, 1024, 16, torch.bfloat16),   # C5 widths, seq % 8 != 0
        (1, 512, 2048, 32, torch.bfloat16),   # C4 widths
        (1, 256, 4096, 64, torch.bfloat16),   # widest statistics
        (2, 128, 1024, 16, torch.float16),
    ],
)
@pytest.mark.parametrize("layout", ["bhsd", "seq_major"])
def test_fused_equals_norm_then_projection_and_float64(gpu_device, batch, seq, d_model, heads, dtype, layout):
    from solution.kernels.norm.hip_residual import hip_layer_norm
    from solution.kernels.projection.hip_qkv_layout import (
        HIP_INITIAL_NORM_QKV_BACKEND,
        hip_qkv_native_bhsd,
        prevalidated_hip_initial_norm_qkv_native_bhsd,
    )

    print(f"norm+qkv B{batch} S{seq} D{d_model} H{heads} {dtype} {layout}", flush=True)
    host, (x, w, b, ln_w, ln_b) = _operands(batch, seq, d_model, dtype, seed=seq + d_model, device=gpu_device)
    norm = _layer_norm(ln_w, ln_b, gpu_device)
    with torch.inference_mode():
        fused = prevalidated_hip_initial_norm_qkv_native_bhsd(x, norm, w, b, num_heads=heads, value_layout=layout)
        normalized, _ = hip_layer_norm(x, norm, normalized_dtype=dtype)
        unfused = hip_qkv_native_bhsd(normalized, w, b, num_heads=heads, value_layout=layout)
    torch.cuda.synchronize()
    assert fused[3] == HIP_INITIAL_NORM_QKV_BACKEND
    if layout == "seq_major":
        assert fused[2].stride(-2) == 1
    for name, got, want in zip("qkv", fused[:3], unfused[:3]):
        assert got.shape == want.shape and got.stride() == want.stride()
        diff = int((got != want).sum())
        assert diff == 0, f"{name}: {diff} elements differ from sah_norm + sah_qkv_projection"
    ulp = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    for name, got, want in zip("qkv", fused[:3], _float64_reference(*host, heads, norm.eps)):
        got = got.float().cpu()
        result = parity_gate(want.float(), got, dtype)
        err = (got.double() - want).abs()
        bound = 2 * ulp * want.abs() + 2e-3
        print(f"  {name}: max_abs={result.max_abs_error:.3g} failed={result.failed_elements}", flush=True)
        assert result.passed, f"{name}: {result.failed_elements} of {result.total_elements} outside the gate"
        assert bool((err <= bound).all()), f"{name}: error {float((err - bound).max()):.3g} above the ulp bound"


def test_ineligible_inputs_raise(gpu_device):
    from solution.kernels.projection.hip_qkv_layout import (
        can_use_hip_initial_norm_qkv_native_bhsd,
        prevalidated_hip_initial_norm_qkv_native_bhsd,
    )

    _, (x, w, b, ln_w, ln_b) = _operands(1, 64, 512, torch.bfloat16, seed=5, device=gpu_device)
    norm = _layer_norm(ln_w, ln_b, gpu_device)
    with torch.inference_mode():
        assert can_use_hip_initial_norm_qkv_native_bhsd(x, norm, w, b, num_heads=8)
        plain = torch.nn.LayerNorm(512, elementwise_affine=False, device=gpu_device, dtype=torch.bfloat16)
        fp32_norm = torch.nn.LayerNorm(512, device=gpu_device)
        _, (x768, w768, b768, lw768, lb768) = _operands(1, 64, 768, torch.bfloat16, seed=6, device=gpu_device)
        cases = [
            (x, plain, w, b, 8),  # no affine parameters
            (x, fp32_norm, w, b, 8),  # parameters in another dtype
            (x768, _layer_norm(lw768, lb768, gpu_device), w768, b768, 12),  # width without statistics
        ]
        for args in cases:
            assert not can_use_hip_initial_norm_qkv_native_bhsd(*args[:4], num_heads=args[4])
            with pytest.raises(RuntimeError, match="ineligible"):
                prevalidated_hip_initial_norm_qkv_native_bhsd(*args[:4], num_heads=args[4])


class _StateSource(torch.nn.Module):
    def __init__(self, tensors):
        super().__init__()
        self._tensors = tensors

    def state_dict(self, *args, **kwargs):
        return dict(self._tensors)


def _model(config, state, device, program):
    from solution.transformer import UserOptimizedTransformer, copy_model_weights

    model = UserOptimizedTransformer(config)
    copy_model_weights(_StateSource(state), model)
    model = model.to(device=device, dtype=torch.bfloat16).eval()
    model.configure_execution(config=program)
    model.set_execution_observation(True)
    return model


@pytest.mark.parametrize(
    "shape",
    [
        (2, 256, 512, 8, 2048, 2),    # C2 widths
        (1, 300, 1024, 16, 4096, 2),  # C5 widths, ragged length
        (1, 256, 2048, 32, 8192, 1),  # C4 widths
    ],
)
def test_fused_initial_norm_plan_equals_the_unfused_plan(gpu_device, shape):
    from solution.config import InitialNormBackend, QKVMaterialization, hip_config

    batch, seq, width, heads, ffn, layers = shape
    print(f"fused initial norm model {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=97)
    x = generate_input(config, seed=97).to(torch.bfloat16)
    fused = _model(config, state, gpu_device, hip_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD, initial_norm=InitialNormBackend.HIP_FUSED_QKV))
    unfused = _model(config, state, gpu_device, hip_config(qkv=QKVMaterialization.HIP_NATIVE_BHSD))
    with torch.inference_mode():
        got = fused(x.to(gpu_device))
        want = unfused(x.to(gpu_device))
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"{int((got != want).sum())} elements differ from the unfused program"
    description = fused.describe_execution_path()
    observed = description["observed_execution_signature"]
    assert observed == description["expected_execution_signature"]
    assert observed["initial_norm_backend"] == "hip_fused_qkv" and observed["initial_norm_launch"] is None
    reference_path = forward(cast_state(state, torch.bfloat16), x, config).float()
    exact = forward(cast_state(cast_state(state, torch.bfloat16), torch.float32), x.float(), config)
    parity = model_parity(exact, reference_path, got.float().cpu())
    print(f"fused initial norm model {shape}: {parity.summary()}", flush=True)
    assert parity.passed, parity.summary()


def test_streamed_long_sequence_with_the_fused_initial_norm(gpu_device):
    """The streamed long-sequence program (one sequence per microbatch, past
    the attention's 4096-key score-bound threshold) with the fused initial
    norm equals the same program with the separate norm kernel."""

    from solution.config import InitialNormBackend, QKVMaterialization
    from solution.shape14.defaults import hip_streamed_config

    config = TransformerConfig(2, 20000, 1024, 16, 4096, 2, True)
    print(f"streamed fused initial norm {config}", flush=True)
    state = xavier_init_weights(config, seed=31)
    x = generate_input(config, seed=31).to(torch.bfloat16).to(gpu_device)
    native = QKVMaterialization.HIP_NATIVE_BHSD
    fused = _model(config, state, gpu_device, hip_streamed_config(microbatch_size=1, qkv=native, initial_norm=InitialNormBackend.HIP_FUSED_QKV))
    unfused = _model(config, state, gpu_device, hip_streamed_config(microbatch_size=1, qkv=native))
    with torch.inference_mode():
        got = fused(x)
        want = unfused(x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(got).all())
    assert torch.equal(got, want)
    assert fused.describe_execution_path()["runtime_backend"] == "streamed"
