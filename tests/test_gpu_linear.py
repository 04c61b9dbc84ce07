"""GPU parity of the fused Linear + bias + exact-GELU kernel (sah_linear).

Reference: the same op in float64 on the CPU from the same 16-bit operands,
``F.gelu(F.linear(x, w, b), approximate="none")``, i.e. the FFN input half of
the official block (oracle/forward.py, official order).  The kernel rounds an
fp32 result once to the operand dtype, so it must pass the 16-bit gate of
oracle.compare (|err| <= 2e-2 or |err| <= 1e-2 |ref|) elementwise; the tests
also bound the error by a few output ulps, which a dropped bias, a wrong
activation or a transposed operand would far exceed.
"""

from __future__ import annotations


import pytest
import torch
import torch.nn.functional as F

from oracle.compare import parity_gate

pytestmark = pytest.mark.gpu


def _operands(rows, k, n, dtype, seed, device, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g)
    w = (torch.rand(n, k, generator=g) * 2 - 1) * (6.0 / (k + n)) ** 0.5 * 2.0
    b = 0.5 * torch.randn(n, generator=g) if bias else None
    cast = lambda t: None if t is None else t.to(dtype)  # noqa: E731
    x, w, b = cast(x), cast(w), cast(b)
    return (x, w, b), tuple(None if t is None else t.to(device) for t in (x, w, b))


def _reference(x, w, b, gelu):
    y = F.linear(x.double(), w.double(), None if b is None else b.double())
    return F.gelu(y, approximate="none") if gelu else y


def _check(reference, got, dtype, what):
    got = got.float().cpu()
    result = parity_gate(reference.float(), got, dtype)
    err = (got.double() - reference).abs()
    # at most a couple of output ulps (bf16: 2^-8 relative, fp16: 2^-11) plus
    # the fp32 accumulation error
    ulp = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    bound = 2 * ulp * reference.abs() + 1e-3
    print(f"{what}: max_abs={result.max_abs_error:.3g} failed={result.failed_elements}", flush=True)
    assert result.passed, f"{what}: {result.failed_elements} of {result.total_elements} outside the gate"
    assert bool((err <= bound).all()), f"{what}: error {float((err - bound).max()):.3g} above a 2-ulp bound"


@pytest.mark.parametrize(
    "rows,k,n",
    [(1, 512, 2048), (255, 512, 2048), (300, 1024, 4096), (1025, 1024, 4096), (513, 2048, 8192), (700, 4096, 1024)],
)
def test_linear_exact_gelu_matches_float64(gpu_device, rows, k, n):
    from solution.kernels.ffn import prevalidated_hip_linear_exact_gelu

    (x, w, b), (xd, wd, bd) = _operands(rows, k, n, torch.bfloat16, seed=rows + k, device=gpu_device)
    with torch.inference_mode():
        hidden, marker = prevalidated_hip_linear_exact_gelu(xd, wd, bd)
    torch.cuda.synchronize()
    assert marker == "hip_linear_exact_gelu" and hidden.shape == (rows, n) and hidden.dtype == torch.bfloat16
    _check(_reference(x, w, b, True), hidden, torch.bfloat16, f"gelu rows={rows} k={k} n={n}")


@pytest.mark.parametrize("bias", [True, False])
def test_plain_linear_and_fp16(gpu_device, bias):
    from solution.kernels.ffn import prevalidated_hip_linear

    for dtype in (torch.bfloat16, torch.float16):
        (x, w, b), (xd, wd, bd) = _operands(777, 1024, 1024, dtype, seed=5, device=gpu_device, bias=bias)
        with torch.inference_mode():
            out, marker = prevalidated_hip_linear(xd, wd, bd)
        torch.cuda.synchronize()
        assert marker == "hip_linear"
        _check(_reference(x, w, b, False), out, dtype, f"linear bias={bias} {dtype}")


def test_strided_rows_and_untouched_tail_through_the_c_abi(gpu_device):
    """x with a padded row stride, y with a wider row stride and rows past the
    last one: the kernel reads only valid rows and writes only [rows, n]."""

    from solution.kernels.hip import _library

    rows, k, n, ldx, ldy = 333, 1024, 2048, 1024 + 64, 2048 + 256
    (x, w, b), (_, wd, bd) = _operands(rows, k, n, torch.bfloat16, seed=9, device=gpu_device)
    xs = torch.full((rows, ldx), float("nan"), dtype=torch.bfloat16)
    xs[:, :k] = x
    xs = xs.to(gpu_device)
    sentinel = -7.0
    y = torch.full((rows + 5, ldy), sentinel, dtype=torch.bfloat16, device=gpu_device)
    lib = _library.load_library()
    status = lib.sah_linear(
        xs.data_ptr(), wd.data_ptr(), bd.data_ptr(), y.data_ptr(), rows, k, n, ldx, ldy,
        _library.dtype_code(torch.bfloat16), _library.SAH_ACTIVATION_GELU_EXACT, 256, 256, 64, 8, 2,
        _library.stream_handle(gpu_device),
    )
    _library.check_status(status, "sah_linear")
    torch.cuda.synchronize()
    y = y.cpu()
    _check(_reference(x, w, b, True), y[:rows, :n], torch.bfloat16, "strided")
    assert bool((y[:rows, n:] == sentinel).all()) and bool((y[rows:] == sentinel).all())


def test_long_sequence_ffn_input_rows_sample(gpu_device):
    """The C5 chunk's FFN input projection (2e5 rows x 1024 -> 4096): rows from
    every part of the output, including the partial last tile, against
    float64, and the full output finite."""

    from solution.kernels.ffn import prevalidated_hip_linear_exact_gelu

    rows, k, n = 200_000, 1024, 4096
    g = torch.Generator(device=gpu_device).manual_seed(3)
    xd = torch.randn(rows, k, device=gpu_device, dtype=torch.bfloat16, generator=g)
    wd = ((torch.rand(n, k, device=gpu_device, generator=g) * 2 - 1) * 0.0765).to(torch.bfloat16)
    bd = (0.5 * torch.randn(n, device=gpu_device, generator=g)).to(torch.bfloat16)
    with torch.inference_mode():
        hidden, _ = prevalidated_hip_linear_exact_gelu(xd, wd, bd)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(hidden).all())
    pick = torch.cat([torch.arange(0, 256), torch.randint(0, rows, (256,), generator=torch.Generator().manual_seed(1)),
                      torch.arange(rows - 64, rows)])
    x, w, b = xd[pick.to(gpu_device)].cpu(), wd.cpu(), bd.cpu()
    _check(_reference(x, w, b, True), hidden[pick.to(gpu_device)], torch.bfloat16, "C5 ffn_in sample")


def test_ineligible_inputs_raise(gpu_device):
    from solution.kernels.ffn import can_use_hip_linear_exact_gelu, prevalidated_hip_linear_exact_gelu

    x = torch.zeros(4, 1000, dtype=torch.bfloat16, device=gpu_device)
    w = torch.zeros(2048, 1000, dtype=torch.bfloat16, device=gpu_device)
    b = torch.zeros(2048, dtype=torch.bfloat16, device=gpu_device)
    assert not can_use_hip_linear_exact_gelu(x, w, b)
    with pytest.raises(RuntimeError, match="ineligible"):
        prevalidated_hip_linear_exact_gelu(x, w, b)
    with pytest.raises(ValueError, match="launch"):
        prevalidated_hip_linear_exact_gelu(x, w, b, block_m=128)
