"""GPU parity of the elementwise exact-GELU kernel (sah_gelu).

Reference: GELU in float64 on the CPU of the same 16-bit inputs,
``F.gelu(x.double(), approximate="none")``.  The kernel evaluates GELU in fp32
and rounds once, so every element must be within one output ulp of the
float64 value (plus 1e-6 absolute for results that underflow toward zero) and
pass the 16-bit gate of oracle.compare.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle.compare import parity_gate

pytestmark = pytest.mark.gpu


def _check(x_cpu, got, dtype, what):
    reference = F.gelu(x_cpu.double(), approximate="none")
    got = got.cpu()
    result = parity_gate(reference.float(), got.float(), dtype)
    ulp = 2.0**-7 if dtype == torch.bfloat16 else 2.0**-10  # relative spacing upper bound
    err = (got.double() - reference).abs()
    bound = ulp * reference.abs() + 1e-6
    print(f"{what}: max_abs={result.max_abs_error:.3g} failed={result.failed_elements}", flush=True)
    assert result.passed, f"{what}: {result.failed_elements} outside the gate"
    assert bool((err <= bound).all()), f"{what}: {int((err > bound).sum())} elements above one ulp"


@pytest.mark.parametrize("n", [1, 7, 8, 4095, 3 * 4096 + 5, 1_000_003])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_exact_gelu_matches_float64(gpu_device, n, dtype):
    from solution.kernels.ffn import prevalidated_hip_exact_gelu

    g = torch.Generator().manual_seed(n)
    x = (torch.randn(n, generator=g) * 3).to(dtype)
    x[: min(n, 4)] = torch.tensor([0.0, -0.0, 8.0, -8.0][: min(n, 4)], dtype=dtype)
    with torch.inference_mode():
        y, marker = prevalidated_hip_exact_gelu(x.to(gpu_device))
    torch.cuda.synchronize()
    assert marker == "hip_exact_gelu" and y.dtype == dtype and y.shape == x.shape
    _check(x, y, dtype, f"gelu n={n} {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_negative_tail_within_one_ulp(gpu_device, dtype):
    """v in [-10, -3]: GELU(v) is 1e-23 .. 4e-3, and the result must stay
    within one ulp RELATIVE to float64 exact GELU (no absolute slack beyond
    half the dtype's smallest subnormal step).  An erfc approximation with
    only an absolute error bound fails this by 1-2% below v = -5."""

    from solution.kernels.ffn import prevalidated_hip_exact_gelu

    x = torch.linspace(-10.0, -3.0, 70001).to(dtype)
    with torch.inference_mode():
        y, _ = prevalidated_hip_exact_gelu(x.to(gpu_device))
    torch.cuda.synchronize()
    # v * erfc(-v / sqrt 2) / 2 in float64: torch's float64 GELU forms
    # 1 + erf(v / sqrt 2), which cancels to 0 below v = -8.3
    xd = x.double()
    reference = xd * 0.5 * torch.special.erfc(-xd / math.sqrt(2.0))
    assert bool((reference < 0).all())
    ulp = 2.0**-7 if dtype == torch.bfloat16 else 2.0**-10
    tiny = 2.0**-134 if dtype == torch.bfloat16 else 2.0**-25
    err = (y.cpu().double() - reference).abs()
    rel = (err / reference.abs()).max().item()
    print(f"negative tail {dtype}: max relative error {rel:.3g}", flush=True)
    assert bool((err <= ulp * reference.abs() + tiny).all()), (
        f"{int((err > ulp * reference.abs() + tiny).sum())} tail elements above one ulp (max rel {rel:.3g})")


@pytest.mark.parametrize("launch", [(512, 1), (1024, 2), (4096, 4), (8192, 8), (16384, 4)])
def test_every_launch_and_in_place(gpu_device, launch):
    from solution.kernels.ffn import prevalidated_hip_exact_gelu

    block_size, warps = launch
    x = (torch.randn(3, 1000, 2048, generator=torch.Generator().manual_seed(2)) * 2).to(torch.bfloat16)
    buffer = x.to(gpu_device)
    with torch.inference_mode():
        y, _ = prevalidated_hip_exact_gelu(buffer, block_size=block_size, num_warps=warps, out=buffer)
    torch.cuda.synchronize()
    assert y.data_ptr() == buffer.data_ptr()
    _check(x, y, torch.bfloat16, f"in place {launch}")


def test_long_sequence_ffn_hidden_sample(gpu_device):
    """The C5 chunk's FFN hidden tensor (2e5 x 4096 bf16): finite everywhere
    and one ulp on a sample spanning the whole tensor, including its end."""

    from solution.kernels.ffn import prevalidated_hip_exact_gelu

    rows, width = 200_000, 4096
    g = torch.Generator(device=gpu_device).manual_seed(5)
    x = (torch.randn(rows, width, generator=g, device=gpu_device) * 1.5).to(torch.bfloat16)
    with torch.inference_mode():
        y, _ = prevalidated_hip_exact_gelu(x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all())
    pick = torch.cat([torch.arange(0, 64), torch.randint(0, rows, (128,), generator=torch.Generator().manual_seed(1)),
                      torch.arange(rows - 64, rows)]).to(gpu_device)
    _check(x[pick].cpu(), y[pick], torch.bfloat16, "C5 hidden sample")


def test_ineligible_and_bad_launch_raise(gpu_device):
    from solution.kernels.ffn import can_use_hip_exact_gelu, prevalidated_hip_exact_gelu

    x32 = torch.zeros(16, device=gpu_device)
    assert not can_use_hip_exact_gelu(x32)
    with pytest.raises(RuntimeError, match="ineligible"):
        prevalidated_hip_exact_gelu(x32)
    x = torch.zeros(16, device=gpu_device, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="launch"):
        prevalidated_hip_exact_gelu(x, block_size=256)
    with pytest.raises(RuntimeError, match="output buffer"):
        prevalidated_hip_exact_gelu(x, out=torch.zeros(8, device=gpu_device, dtype=torch.bfloat16))
