"""GPU parity of the whole FFN fused through its residual LayerNorm
(sah_mlp_residual_norm, the HIP_FUSED_MLP_BOUNDARY FFN backend).

Three references:

* The unfused HIP chain on the same operands, ``sah_linear`` with the exact
  GELU epilogue, ``sah_linear`` for the output projection, then
  ``sah_residual_norm``: the same MFMA operand roles, the same ascending
  16-wide K order, the same bias / GELU / rounding points, so the fused
  kernel must equal it bit for bit (residual and normalized).  A wrong W2
  column, a hidden unit of the wrong chunk, a dropped rounding or bias, or a
  norm mapped differently fails this.  (width 256, ffn a multiple of 256:
  the shapes sah_linear serves.)
* float64 on the CPU with the kernel's rounding points (hidden, update,
  residual to the stream dtype), every shape including width 128: residual
  within a few ulps, normalized within the 16-bit gate.
* The whole model against the CPU oracle (model-level accuracy rule), with
  the observed execution equal to the plan's expected trace.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle.compare import model_parity, parity_gate
from oracle.forward import TransformerConfig, cast_state, forward, generate_input, xavier_init_weights

pytestmark = pytest.mark.gpu


def _layer_norm(width, dtype, device, seed):
    ln = torch.nn.LayerNorm(width).to(device=device, dtype=dtype)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        ln.weight.copy_((1 + 0.25 * torch.randn(width, generator=g)).to(dtype))
        ln.bias.copy_((0.1 * torch.randn(width, generator=g)).to(dtype))
    return ln


def _operands(rows, width, ffn, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, rows, width, generator=g).to(dtype)
    w1 = ((torch.rand(ffn, width, generator=g) * 2 - 1) * (6.0 / (width + ffn)) ** 0.5 * 2).to(dtype)
    b1 = (0.2 * torch.randn(ffn, generator=g)).to(dtype)
    w2 = ((torch.rand(width, ffn, generator=g) * 2 - 1) * (6.0 / (width + ffn)) ** 0.5).to(dtype)
    b2 = (0.1 * torch.randn(width, generator=g)).to(dtype)
    value = (2.0 * torch.randn(1, rows, width, generator=g)).to(dtype)
    return x, w1, b1, w2, b2, value


def _ulp(t: torch.Tensor, dtype) -> torch.Tensor:
    mant = 8 if dtype == torch.bfloat16 else 11
    exponent = torch.floor(torch.log2(t.abs().clamp_min(2.0**-100)))
    return torch.pow(2.0, exponent - (mant - 1))


@pytest.mark.parametrize("rows,ffn", [(1000, 1024), (77, 256), (64, 2048)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_mlp_equals_the_unfused_hip_chain_bitwise(gpu_device, rows, ffn, dtype):
    from solution.kernels.boundary.hip_mlp_residual_norm import hip_mlp_residual_norm
    from solution.kernels.hip._library import SAH_ACTIVATION_GELU_EXACT, check_status, dtype_code, load_library
    from solution.kernels.norm.hip_residual import hip_residual_layer_norm

    width = 256
    print(f"fused MLP vs unfused HIP chain rows {rows} ffn {ffn} {dtype}", flush=True)
    host = _operands(rows, width, ffn, dtype, seed=rows + ffn)
    x, w1, b1, w2, b2, value = (t.to(gpu_device) for t in host)
    ln = _layer_norm(width, dtype, gpu_device, seed=5)
    lib = load_library()
    with torch.inference_mode():
        r_fused, y_fused, marker = hip_mlp_residual_norm(x, w1, b1, w2, b2, value, ln)
        hidden = torch.empty(1, rows, ffn, device=gpu_device, dtype=dtype)
        update = torch.empty_like(value)
        for src, w, b, out, n, k, act in (
            (x, w1, b1, hidden, ffn, width, SAH_ACTIVATION_GELU_EXACT),
            (hidden, w2, b2, update, width, ffn, 0),
        ):
            status = lib.sah_linear(src.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr(), rows, k, n, k, n,
                                    dtype_code(dtype), act, 256, 256, 64, 8, 2, None)
            check_status(status, "sah_linear")
        r_ref, y_ref, _ = hip_residual_layer_norm(value, update, ln)
    torch.cuda.synchronize()
    assert marker == "hip_mlp_residual_norm"
    assert torch.equal(r_fused, r_ref), f"residual: {int((r_fused != r_ref).sum())} elements differ"
    assert torch.equal(y_fused, y_ref), f"normalized: {int((y_fused != y_ref).sum())} elements differ"


@pytest.mark.parametrize("width,ffn,rows", [(128, 128, 1000), (128, 512, 33), (256, 1024, 300), (256, 64, 129)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_random_operands_match_float64(gpu_device, width, ffn, rows, dtype):
    from solution.kernels.boundary.hip_mlp_residual_norm import hip_mlp_residual_norm

    print(f"fused MLP vs float64 width {width} ffn {ffn} rows {rows} {dtype}", flush=True)
    x, w1, b1, w2, b2, value = _operands(rows, width, ffn, dtype, seed=width + ffn + rows)
    ln = _layer_norm(width, dtype, gpu_device, seed=rows)
    with torch.inference_mode():
        r, y, _ = hip_mlp_residual_norm(*(t.to(gpu_device) for t in (x, w1, b1, w2, b2, value)), ln)
    torch.cuda.synchronize()
    r, y = r.double().cpu(), y.double().cpu()
    pre = x.double() @ w1.double().T + b1.double()
    hidden = (pre * 0.5 * torch.special.erfc(-pre / 2.0**0.5)).to(dtype)
    u64 = hidden.double() @ w2.double().T + b2.double()
    r_ref = (value.double() + u64.to(dtype).double()).to(dtype).double()
    # A hidden element that the fp32 accumulation rounds the other way moves
    # the update by one ulp of that element times |w2|: an absolute amount,
    # bounded per row by the largest hidden ulp times the largest |w2| of the
    # column (a few such elements per row at most).
    flip = _ulp(hidden.double(), dtype).amax(-1, keepdim=True) * w2.double().abs().amax(-1)
    slack = 4 * _ulp(u64, dtype) + 4 * _ulp(r_ref, dtype) + 3 * flip
    excess = (r - r_ref).abs() - slack
    print(f"  residual max excess over slack {float(excess.max()):.3g}", flush=True)
    assert bool((excess <= 0).all())
    y64 = F.layer_norm(r, (width,), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    result = parity_gate(y64.float(), y.float(), dtype)
    print(f"  normalized max_abs={result.max_abs_error:.3g} failed={result.failed_elements}", flush=True)
    assert result.passed
    assert bool(((y - y64).abs() <= 2 * _ulp(y64, dtype) + 1e-3).all())


def test_normalized_is_the_fused_norm_of_the_residual(gpu_device):
    """The epilogue's norm arithmetic and lane mapping are the fused norm
    kernel's: normalizing the kernel's own residual with sah_norm gives its
    normalized output bit for bit (width 128 and 256)."""

    from solution.kernels.boundary.hip_mlp_residual_norm import hip_mlp_residual_norm
    from solution.kernels.norm.hip_residual import hip_layer_norm

    for width, ffn in ((128, 384), (256, 512)):
        x, w1, b1, w2, b2, value = (t.to(gpu_device) for t in _operands(513, width, ffn, torch.bfloat16, seed=width))
        ln = _layer_norm(width, torch.bfloat16, gpu_device, seed=3)
        with torch.inference_mode():
            r, y, _ = hip_mlp_residual_norm(x, w1, b1, w2, b2, value, ln)
            y_norm, _ = hip_layer_norm(r, ln, normalized_dtype=torch.bfloat16)
        assert torch.equal(y, y_norm), f"width {width}"


def test_ineligible_inputs_raise(gpu_device):
    from solution.kernels.boundary.hip_mlp_residual_norm import (
        can_use_hip_mlp_residual_norm,
        hip_mlp_residual_norm,
    )

    x, w1, b1, w2, b2, value = (t.to(gpu_device) for t in _operands(64, 256, 512, torch.bfloat16, seed=1))
    ln = _layer_norm(256, torch.bfloat16, gpu_device, seed=1)
    with torch.inference_mode():
        assert can_use_hip_mlp_residual_norm(x, w1, b1, w2, b2, value, ln)
        bad = [
            (x.float(), w1, b1, w2, b2, value, ln),            # mixed dtypes
            (x, w1[:500], b1[:500], w2[:, :500], b2, value, ln),  # ffn not a multiple of 64
            (x, w1, b1, w2.t().contiguous().t(), b2, value, ln),  # W2 not contiguous
            (x, w1, b1, w2, b2, value, torch.nn.LayerNorm(256, device=gpu_device)),  # fp32 norm params
        ]
        for args in bad:
            assert not can_use_hip_mlp_residual_norm(*args)
            with pytest.raises(RuntimeError, match="ineligible"):
                hip_mlp_residual_norm(*args)


class _StateSource(torch.nn.Module):
    def __init__(self, tensors):
        super().__init__()
        self._tensors = tensors

    def state_dict(self, *args, **kwargs):
        return dict(self._tensors)


@pytest.mark.parametrize(
    "shape",
    [
        (4, 256, 256, 4, 1024, 2),  # width 256
        (8, 128, 128, 2, 128, 2),   # the reference's D = F = 128
    ],
)
def test_fused_mlp_program_matches_the_oracle(gpu_device, shape):
    from solution.config import FFNBackend, hip_config
    from solution.transformer import UserOptimizedTransformer, copy_model_weights

    batch, seq, width, heads, ffn, layers = shape
    print(f"fused MLP model {shape}", flush=True)
    config = TransformerConfig(batch, seq, width, heads, ffn, layers, True)
    state = xavier_init_weights(config, seed=11)
    x = generate_input(config, seed=11).to(torch.bfloat16)
    model = UserOptimizedTransformer(config)
    copy_model_weights(_StateSource(state), model)
    model = model.to(device=gpu_device, dtype=torch.bfloat16).eval()
    model.configure_execution(config=hip_config(ffn=FFNBackend.HIP_FUSED_MLP_BOUNDARY))
    model.set_execution_observation(True)
    with torch.inference_mode():
        output = model(x.to(gpu_device))
    torch.cuda.synchronize()
    description = model.describe_execution_path()
    observed = description["observed_execution_signature"]
    assert observed == description["expected_execution_signature"]
    assert observed["ffn_backend"] == "hip_fused_mlp_boundary" and observed["complete"]
    reference_path = forward(cast_state(state, torch.bfloat16), x, config).float()
    exact = forward(cast_state(cast_state(state, torch.bfloat16), torch.float32), x.float(), config)
    parity = model_parity(exact, reference_path, output.float().cpu())
    print(f"fused MLP model {shape}: {parity.summary()}", flush=True)
    assert parity.passed, parity.summary()


@pytest.mark.parametrize("width,ffn", [(128, 384), (256, 512)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rms_mode_through_the_c_abi(gpu_device, width, ffn, dtype):
    """sah_mlp_residual_norm with SAH_NORM_RMS (called through ctypes; the
    model wrapper passes SAH_NORM_LAYER): the residual equals the LayerNorm
    mode's bit for bit (the FFN and the add do not depend on the norm), and
    the normalized output equals sah_norm's RMSNorm of that residual bit for
    bit, at widths 128 and 256; and it is within the 16-bit gate of float64
    RMSNorm, x * rsqrt(mean(x^2) + eps) * gamma."""

    from solution.kernels.boundary.hip_mlp_residual_norm import BLOCK_ROWS, NUM_WARPS, hip_mlp_residual_norm
    from solution.kernels.hip._library import SAH_NORM_RMS, check_status, dtype_code, load_library, stream_handle
    from solution.kernels.norm.hip_residual import hip_rms_norm

    rows = 515
    print(f"fused MLP RMS mode width {width} ffn {ffn} {dtype}", flush=True)
    x, w1, b1, w2, b2, value = (t.to(gpu_device) for t in _operands(rows, width, ffn, dtype, seed=width + 7))
    ln = _layer_norm(width, dtype, gpu_device, seed=9)
    rms = torch.nn.RMSNorm(width, eps=1e-5).to(device=gpu_device, dtype=dtype)
    with torch.no_grad():
        rms.weight.copy_(ln.weight)
    residual = torch.empty_like(value)
    normalized = torch.empty_like(value)
    with torch.inference_mode():
        r_layer, _, _ = hip_mlp_residual_norm(x, w1, b1, w2, b2, value, ln)
        status = load_library().sah_mlp_residual_norm(
            x.data_ptr(), w1.data_ptr(), b1.data_ptr(), w2.data_ptr(), b2.data_ptr(), value.data_ptr(),
            rms.weight.data_ptr(), None, residual.data_ptr(), normalized.data_ptr(),
            rows, width, ffn, width, 1e-5, dtype_code(dtype), SAH_NORM_RMS, BLOCK_ROWS, NUM_WARPS,
            stream_handle(gpu_device),
        )
        check_status(status, "sah_mlp_residual_norm (RMS)")
        y_rms, _ = hip_rms_norm(residual, rms.weight, eps=1e-5, normalized_dtype=dtype)
    torch.cuda.synchronize()
    assert torch.equal(residual, r_layer), f"residual: {int((residual != r_layer).sum())} elements differ"
    assert torch.equal(normalized, y_rms), f"normalized: {int((normalized != y_rms).sum())} elements differ"
    r64 = residual.double().cpu()
    y64 = r64 * torch.rsqrt((r64 * r64).mean(-1, keepdim=True) + 1e-5) * rms.weight.double().cpu()
    result = parity_gate(y64.float(), normalized.float().cpu(), dtype)
    print(f"  RMS normalized vs float64: max_abs={result.max_abs_error:.3g} failed={result.failed_elements}",
          flush=True)
    assert result.passed
