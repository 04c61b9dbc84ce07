"""GPU parity of the fused Linear + residual + LayerNorm boundary
(sah_linear_residual_norm, the linear-boundary residual-norm backend).

Two references:

* Exact products.  With small-integer x and W every product and partial sum
  is exact in fp32, so the update round(x W^T + b) is known exactly whatever
  the accumulation order.  The fused kernel must then equal the unfused
  boundary (the HIP residual norm, whose arithmetic it shares) applied to
  that update, bit for bit: residual and normalized.  A dropped bias, a wrong
  K permutation, a wrong row or column of the update, or a norm that differs
  from the unfused one in any element fails this.
* Random operands against float64: update, residual and LayerNorm computed in
  float64 from the same 16-bit operands with the kernel's roundings (update,
  then residual, to the stream dtype); residual within one ulp, normalized
  within the 16-bit gate of oracle.compare and a few ulps.
"""

from __future__ import annotations


import pytest
import torch
import torch.nn.functional as F

from oracle.compare import parity_gate

pytestmark = pytest.mark.gpu


def _layer_norm(width, dtype, device, seed, affine=True):
    ln = torch.nn.LayerNorm(width).to(device=device, dtype=dtype)
    if affine:
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            ln.weight.copy_((1 + 0.25 * torch.randn(width, generator=g)).to(dtype))
            ln.bias.copy_((0.1 * torch.randn(width, generator=g)).to(dtype))
    return ln


def _ulp(t: torch.Tensor, dtype) -> torch.Tensor:
    mant = 8 if dtype == torch.bfloat16 else 11
    exponent = torch.floor(torch.log2(t.abs().clamp_min(2.0**-100)))
    return torch.pow(2.0, exponent - (mant - 1))


@pytest.mark.parametrize("width,in_features,batch,seq", [
    (1024, 1024, 2, 200),    # attention output projection, long-sequence widths
    (1024, 4096, 1, 130),    # FFN output projection (ragged rows)
    (512, 512, 4, 256),      # short-sequence widths
    (512, 2048, 3, 77),      # short-sequence FFN output projection, ragged
])
def test_exact_products_match_the_unfused_boundary_bitwise(gpu_device, width, in_features, batch, seq):
    from solution.kernels.boundary import block_rows_for, hip_linear_residual_norm
    from solution.kernels.norm.hip_residual import hip_residual_layer_norm

    print(f"exact boundary width {width} in {in_features} B{batch} S{seq}", flush=True)
    g = torch.Generator().manual_seed(width + in_features + seq)
    dtype = torch.bfloat16
    x = torch.randint(-2, 3, (batch, seq, in_features), generator=g).to(dtype)
    w = (torch.randint(-2, 3, (width, in_features), generator=g).float() / 16).to(dtype)
    b = (torch.randint(-64, 65, (width,), generator=g).float() / 8).to(dtype)
    value = torch.randn(batch, seq, width, generator=g).to(dtype)
    # fp32-exact update, one rounding
    update = (x.double() @ w.double().T + b.double()).to(dtype)
    xd, wd, bd, vd, ud = (t.to(gpu_device) for t in (x, w, b, value, update))
    ln = _layer_norm(width, dtype, gpu_device, seed=7)
    with torch.inference_mode():
        r_fused, y_fused, marker = hip_linear_residual_norm(
            xd, wd, bd, vd, ln, block_rows=block_rows_for(width), num_warps=8)
        r_ref, y_ref, _ = hip_residual_layer_norm(vd, ud, ln, block_rows=8, num_warps=8)
    torch.cuda.synchronize()
    assert marker == "hip_linear_residual_norm"
    assert torch.equal(r_fused, r_ref), "residual differs from the unfused boundary"
    assert torch.equal(y_fused, y_ref), "normalized differs from the unfused boundary"


@pytest.mark.parametrize("width,in_features,rows", [(1024, 1024, 300), (1024, 4096, 64), (512, 2048, 1000)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_random_operands_match_float64(gpu_device, width, in_features, rows, dtype):
    from solution.kernels.boundary import block_rows_for, hip_linear_residual_norm

    print(f"random boundary width {width} in {in_features} rows {rows} {dtype}", flush=True)
    g = torch.Generator().manual_seed(rows + width)
    x = torch.randn(1, rows, in_features, generator=g).to(dtype)
    w = ((torch.rand(width, in_features, generator=g) * 2 - 1) * (6.0 / (width + in_features)) ** 0.5).to(dtype)
    b = (0.1 * torch.randn(width, generator=g)).to(dtype)
    value = (2.0 * torch.randn(1, rows, width, generator=g)).to(dtype)
    ln = _layer_norm(width, dtype, gpu_device, seed=rows)
    with torch.inference_mode():
        r, y, _ = hip_linear_residual_norm(
            x.to(gpu_device), w.to(gpu_device), b.to(gpu_device), value.to(gpu_device), ln,
            block_rows=block_rows_for(width), num_warps=8)
    torch.cuda.synchronize()
    r, y = r.double().cpu(), y.double().cpu()
    u64 = x.double() @ w.double().T + b.double()
    r_ref = (value.double() + u64.to(dtype).double()).to(dtype).double()
    # the kernel's fp32 accumulation may round the update one ulp the other way
    assert bool(((r - r_ref).abs() <= _ulp(r_ref, dtype) * 1.01 + _ulp(u64, dtype)).all())
    y64 = F.layer_norm(r, (width,), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    result = parity_gate(y64.float(), y.float(), dtype)
    print(f"  normalized max_abs={result.max_abs_error:.3g} failed={result.failed_elements}", flush=True)
    assert result.passed
    # y of the kernel's own residual: rounding of y plus fp32 statistics
    y_own = F.layer_norm(r, (width,), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    assert bool(((y - y_own).abs() <= 2 * _ulp(y_own, dtype) + 1e-3).all())


def test_strided_rows_null_params_and_rms_through_the_c_abi(gpu_device):
    """x with a padded row stride, no bias / gamma / beta, RMS statistics;
    rows past the last one untouched."""

    from solution.kernels.hip import _library

    width, in_features, rows, ldx = 1024, 1024, 100, 1024 + 64
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(3)
    x = torch.randint(-2, 3, (rows, in_features), generator=g).to(dtype)
    w = (torch.randint(-2, 3, (width, in_features), generator=g).float() / 16).to(dtype)
    value = torch.randn(rows, width, generator=g).to(dtype)
    xs = torch.full((rows, ldx), float("nan"), dtype=dtype)
    xs[:, :in_features] = x
    sentinel = -5.0
    residual = torch.full((rows + 3, width), sentinel, dtype=dtype, device=gpu_device)
    normalized = torch.full((rows + 3, width), sentinel, dtype=dtype, device=gpu_device)
    xs, wd, vd = xs.to(gpu_device), w.to(gpu_device), value.to(gpu_device)
    lib = _library.load_library()
    status = lib.sah_linear_residual_norm(
        xs.data_ptr(), wd.data_ptr(), None, vd.data_ptr(), None, None, residual.data_ptr(),
        normalized.data_ptr(), rows, in_features, width, ldx, 1e-5, _library.dtype_code(dtype),
        _library.SAH_NORM_RMS, 64, 8, _library.stream_handle(gpu_device))
    _library.check_status(status, "sah_linear_residual_norm")
    torch.cuda.synchronize()
    residual, normalized = residual.cpu(), normalized.cpu()
    update = (x.double() @ w.double().T).to(dtype)
    r_ref = (value.float() + update.float()).to(dtype)
    assert torch.equal(residual[:rows], r_ref)
    rr = r_ref.double()
    y_ref = rr * torch.rsqrt((rr * rr).mean(-1, keepdim=True) + 1e-5)
    assert parity_gate(y_ref.float(), normalized[:rows].float(), dtype).passed
    assert bool((residual[rows:] == sentinel).all()) and bool((normalized[rows:] == sentinel).all())


def test_output_buffer_and_long_sequence_chunk_sample(gpu_device):
    """The long-sequence chunk's FFN output boundary (2e5 rows, 4096 -> 1024)
    writing into a caller's buffer: finite everywhere, sampled rows against
    float64."""

    from solution.kernels.boundary import block_rows_for, hip_linear_residual_norm

    rows, width, in_features, dtype = 200_000, 1024, 4096, torch.bfloat16
    g = torch.Generator(device=gpu_device).manual_seed(11)
    x = torch.randn(2, rows // 2, in_features, device=gpu_device, generator=g).to(dtype)
    w = ((torch.rand(width, in_features, device=gpu_device, generator=g) * 2 - 1) * 0.034).to(dtype)
    b = (0.1 * torch.randn(width, device=gpu_device, generator=g)).to(dtype)
    value = torch.randn(2, rows // 2, width, device=gpu_device, generator=g).to(dtype)
    ln = _layer_norm(width, dtype, gpu_device, seed=5)
    out = torch.empty(2, rows // 2, width, device=gpu_device, dtype=dtype)
    with torch.inference_mode():
        r, y, _ = hip_linear_residual_norm(x, w, b, value, ln, block_rows=block_rows_for(width), num_warps=8, out=out)
    torch.cuda.synchronize()
    assert y.data_ptr() == out.data_ptr()
    assert bool(torch.isfinite(y).all()) and bool(torch.isfinite(r).all())
    pick = torch.cat([torch.arange(0, 64), torch.arange(rows // 2 - 32, rows // 2 + 32), torch.arange(rows - 64, rows)])
    xf, vf, rf, yf = (t.reshape(rows, -1)[pick.to(gpu_device)].double().cpu() for t in (x, value, r, y))
    u = (xf @ w.double().cpu().T + b.double().cpu()).to(dtype).double()
    r_ref = (vf + u).to(dtype).double()
    assert bool(((rf - r_ref).abs() <= _ulp(r_ref, dtype) * 1.01 + _ulp(u, dtype)).all())
    y_ref = F.layer_norm(r_ref, (width,), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    assert parity_gate(y_ref.float(), yf.float(), dtype).passed


def test_ineligible_inputs_raise(gpu_device):
    from solution.kernels.boundary import can_use_hip_linear_residual_norm, hip_linear_residual_norm

    dtype = torch.bfloat16
    with torch.inference_mode():
        x = torch.zeros(2, 8, 768, dtype=dtype, device=gpu_device)
        w = torch.zeros(768, 768, dtype=dtype, device=gpu_device)
        v = torch.zeros(2, 8, 768, dtype=dtype, device=gpu_device)
        ln = torch.nn.LayerNorm(768).to(gpu_device, dtype)
        assert not can_use_hip_linear_residual_norm(x, w, None, v, ln, block_rows=85, num_warps=8)
        with pytest.raises(RuntimeError, match="ineligible"):
            hip_linear_residual_norm(x, w, None, v, ln, block_rows=85, num_warps=8)
        x = torch.zeros(2, 8, 1024, dtype=dtype, device=gpu_device)
        w = torch.zeros(1024, 1024, dtype=dtype, device=gpu_device)
        v = torch.zeros(2, 8, 1024, dtype=dtype, device=gpu_device)
        ln = torch.nn.LayerNorm(1024).to(gpu_device, dtype)
        assert can_use_hip_linear_residual_norm(x, w, None, v, ln, block_rows=64, num_warps=8)
        assert not can_use_hip_linear_residual_norm(x, w, None, v, ln, block_rows=32, num_warps=8)
        assert not can_use_hip_linear_residual_norm(x, w, None, v.float(), ln, block_rows=64, num_warps=8)
        with pytest.raises(RuntimeError, match="output buffer"):
            hip_linear_residual_norm(x, w, None, v, ln, block_rows=64, num_warps=8, out=torch.empty_like(v).float())
    assert not can_use_hip_linear_residual_norm(x, w, None, v, ln, block_rows=64, num_warps=8)  # grad enabled
