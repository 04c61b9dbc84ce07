"""GPU parity of the packed QKV projection with the head-major epilogue
(sah_qkv_projection, the native-layout QKV path).

Reference: the same op in float64 on the CPU from the same 16-bit operands,
``F.linear(x, W_qkv, b_qkv)`` split into query / key / value and each viewed
as [B, H, S, head_dim] -- the official model's separate q/k/v projections
(oracle/forward.py) with the packed weight of copy_model_weights.  The kernel
rounds an fp32 result once to the operand dtype, so every element must pass
the 16-bit gate of oracle.compare and lie within a couple of output ulps of
the float64 value; a transposed operand, a dropped bias, a q/k/v block or head
written to the wrong place, or a token mapped to the wrong sequence fails
both by far.
"""

from __future__ import annotations


import pytest
import torch
import torch.nn.functional as F

from oracle.compare import parity_gate

pytestmark = pytest.mark.gpu


def _operands(batch, seq, d_model, dtype, seed, device):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, seq, d_model, generator=g)
    w = (torch.rand(3 * d_model, d_model, generator=g) * 2 - 1) * (6.0 / (4 * d_model)) ** 0.5 * 2.0
    b = 0.5 * torch.randn(3 * d_model, generator=g)
    x, w, b = (t.to(dtype) for t in (x, w, b))
    return (x, w, b), tuple(t.to(device) for t in (x, w, b))


def _reference(x, w, b, heads):
    batch, seq, d_model = x.shape
    packed = F.linear(x.double(), w.double(), b.double())
    parts = packed.split(d_model, dim=-1)
    return tuple(p.reshape(batch, seq, heads, d_model // heads).transpose(1, 2) for p in parts)


def _check(reference, got, dtype, what):
    got = got.float().cpu()
    assert got.shape == reference.shape, f"{what}: shape {tuple(got.shape)} != {tuple(reference.shape)}"
    result = parity_gate(reference.float(), got, dtype)
    err = (got.double() - reference).abs()
    ulp = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    bound = 2 * ulp * reference.abs() + 1e-3
    print(f"{what}: max_abs={result.max_abs_error:.3g} failed={result.failed_elements}", flush=True)
    assert result.passed, f"{what}: {result.failed_elements} of {result.total_elements} outside the gate"
    assert bool((err <= bound).all()), f"{what}: error {float((err - bound).max()):.3g} above a 2-ulp bound"


@pytest.mark.parametrize(
    "batch,seq,d_model,heads",
    [
        (2, 256, 512, 8),     # short-sequence widths; tiles hold whole sequences
        (1, 300, 1024, 16),   # long-sequence widths; ragged length (seq % 8 != 0)
        (3, 24, 256, 4),      # tiles spanning many short sequences
        (2, 40, 512, 4),      # head_dim 128
        (1, 512, 2048, 32),   # config-4 widths
        (5, 1000, 1024, 16),  # rows not a multiple of the tile, seq % 8 == 0
    ],
)
@pytest.mark.parametrize("layout", ["bhsd", "seq_major"])
def test_native_qkv_matches_float64(gpu_device, batch, seq, d_model, heads, layout):
    from solution.kernels.projection import HIP_QKV_NATIVE_BHSD_BACKEND, hip_qkv_native_bhsd

    print(f"qkv B{batch} S{seq} D{d_model} H{heads} {layout}", flush=True)
    (x, w, b), (xd, wd, bd) = _operands(batch, seq, d_model, torch.bfloat16, seed=seq + d_model, device=gpu_device)
    with torch.inference_mode():
        q, k, v, marker = hip_qkv_native_bhsd(xd, wd, bd, num_heads=heads, value_layout=layout)
    torch.cuda.synchronize()
    assert marker == HIP_QKV_NATIVE_BHSD_BACKEND
    assert q.is_contiguous() and k.is_contiguous()
    if layout == "seq_major":
        assert v.stride(-2) == 1 and v.stride(-1) >= seq and v.stride(-1) % 8 == 0
    else:
        assert v.is_contiguous()
    for name, ref, got in zip("qkv", _reference(x, w, b, heads), (q, k, v)):
        _check(ref, got, torch.bfloat16, f"{name} B{batch} S{seq} D{d_model} {layout}")


def test_fp16_operands(gpu_device):
    from solution.kernels.projection import hip_qkv_native_bhsd

    (x, w, b), (xd, wd, bd) = _operands(2, 136, 512, torch.float16, seed=3, device=gpu_device)
    with torch.inference_mode():
        q, k, v, _ = hip_qkv_native_bhsd(xd, wd, bd, num_heads=8, value_layout="seq_major")
    torch.cuda.synchronize()
    for name, ref, got in zip("qkv", _reference(x, w, b, 8), (q, k, v)):
        _check(ref, got, torch.float16, f"fp16 {name}")


def test_strided_rows_and_untouched_padding_through_the_c_abi(gpu_device):
    """x with a padded row stride, a V^T buffer with a wider seq stride: the
    kernel reads only the valid columns and writes only tokens [0, S) of each
    V^T row, and no bias (NULL) means zero bias."""

    from solution.kernels.hip import _library

    batch, seq, d_model, heads, ldx, ldv = 2, 200, 1024, 16, 1024 + 64, 200 + 24
    hd = d_model // heads
    (x, w, _), (_, wd, _) = _operands(batch, seq, d_model, torch.bfloat16, seed=9, device=gpu_device)
    xs = torch.full((batch * seq, ldx), float("nan"), dtype=torch.bfloat16)
    xs[:, :d_model] = x.reshape(batch * seq, d_model)
    xs = xs.to(gpu_device)
    sentinel = -7.0
    q = torch.full((batch, heads, seq, hd), sentinel, dtype=torch.bfloat16, device=gpu_device)
    k = torch.full_like(q, sentinel)
    vt = torch.full((batch, heads, hd, ldv), sentinel, dtype=torch.bfloat16, device=gpu_device)
    lib = _library.load_library()
    status = lib.sah_qkv_projection(
        xs.data_ptr(), wd.data_ptr(), None, q.data_ptr(), k.data_ptr(), vt.data_ptr(),
        batch, seq, d_model, heads, ldx, _library.SAH_QKV_VALUE_SEQ_MAJOR, ldv,
        _library.dtype_code(torch.bfloat16), 256, 256, 64, 8, _library.stream_handle(gpu_device),
    )
    _library.check_status(status, "sah_qkv_projection")
    torch.cuda.synchronize()
    rq, rk, rv = _reference(x, w, torch.zeros(3 * d_model, dtype=torch.bfloat16), heads)
    _check(rq, q, torch.bfloat16, "strided q")
    _check(rk, k, torch.bfloat16, "strided k")
    vt = vt.cpu()
    _check(rv, vt[..., :seq].transpose(-1, -2), torch.bfloat16, "strided v")
    assert bool((vt[..., seq:] == sentinel).all()), "padding tokens of V^T were written"


def test_seq_major_value_feeds_the_attention_bitwise(gpu_device):
    """The attention reads the head_dim-contiguous value as given; the
    seq-contiguous value it first copies key-major into its workspace.  Both
    paths give the same V operand, so the outputs are bitwise equal."""

    from solution.kernels.projection import hip_qkv_native_bhsd
    from solution.shape14.hip_streaming_dh64 import prevalidated_hip_streaming_dh64_causal_attention_bsd

    batch, seq, d_model, heads = 2, 1000, 1024, 16
    _, (xd, wd, bd) = _operands(batch, seq, d_model, torch.bfloat16, seed=21, device=gpu_device)
    with torch.inference_mode():
        q, k, v_t, _ = hip_qkv_native_bhsd(xd, wd, bd, num_heads=heads, value_layout="seq_major")
        q2, k2, v, _ = hip_qkv_native_bhsd(xd, wd, bd, num_heads=heads, value_layout="bhsd")
        assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v_t, v)
        direct, _ = prevalidated_hip_streaming_dh64_causal_attention_bsd(q, k, v_t, block_m=128, num_warps=4)
        transposed, _ = prevalidated_hip_streaming_dh64_causal_attention_bsd(q, k, v, block_m=128, num_warps=4)
    torch.cuda.synchronize()
    assert torch.equal(direct, transposed)


def test_long_sequence_chunk_rows_sample(gpu_device):
    """The long-sequence chunk's projection (2 x 100000 tokens, D 1024, 16
    heads) with the seq-major value: tokens from the start, the middle, both
    sides of the sequence boundary and the end, against float64."""

    from solution.kernels.projection import hip_qkv_native_bhsd

    batch, seq, d_model, heads = 2, 100_000, 1024, 16
    g = torch.Generator(device=gpu_device).manual_seed(5)
    xd = torch.randn(batch, seq, d_model, device=gpu_device, dtype=torch.bfloat16, generator=g)
    wd = ((torch.rand(3 * d_model, d_model, device=gpu_device, generator=g) * 2 - 1) * 0.0541).to(torch.bfloat16)
    bd = (0.5 * torch.randn(3 * d_model, device=gpu_device, generator=g)).to(torch.bfloat16)
    with torch.inference_mode():
        q, k, v, _ = hip_qkv_native_bhsd(xd, wd, bd, num_heads=heads, value_layout="seq_major")
    torch.cuda.synchronize()
    assert all(bool(torch.isfinite(t).all()) for t in (q, k, v))
    tokens = torch.cat([torch.arange(0, 64), torch.arange(seq // 2 - 32, seq // 2 + 32),
                        torch.arange(seq - 64, seq), torch.randint(0, seq, (64,), generator=torch.Generator().manual_seed(2))])
    for bi in range(batch):
        x = xd[bi, tokens.to(gpu_device)].cpu().unsqueeze(0)
        rq, rk, rv = _reference(x, wd.cpu(), bd.cpu(), heads)
        sel = tokens.to(gpu_device)
        for name, ref, got in zip("qkv", (rq, rk, rv), (q, k, v)):
            _check(ref[0], got[bi][:, sel], torch.bfloat16, f"C5 chunk {name} batch {bi}")


def test_ineligible_inputs_raise(gpu_device):
    from solution.kernels.projection import (
        can_use_hip_qkv_native_bhsd,
        hip_qkv_native_bhsd,
        prevalidated_hip_qkv_native_bhsd,
    )

    with torch.inference_mode():
        x = torch.zeros(2, 16, 640, dtype=torch.bfloat16, device=gpu_device)
        w = torch.zeros(1920, 640, dtype=torch.bfloat16, device=gpu_device)
        b = torch.zeros(1920, dtype=torch.bfloat16, device=gpu_device)
        assert not can_use_hip_qkv_native_bhsd(x, w, b, num_heads=10)
        with pytest.raises(RuntimeError, match="ineligible"):
            hip_qkv_native_bhsd(x, w, b, num_heads=10)
        with pytest.raises(RuntimeError, match="ineligible"):
            prevalidated_hip_qkv_native_bhsd(x, w, b, num_heads=10)
        x = torch.zeros(2, 16, 512, dtype=torch.bfloat16, device=gpu_device)
        w = torch.zeros(1536, 512, dtype=torch.bfloat16, device=gpu_device)
        with pytest.raises(ValueError, match="launch"):
            prevalidated_hip_qkv_native_bhsd(x, w, None, num_heads=8, block_m=64)
        with pytest.raises(ValueError, match="layout"):
            prevalidated_hip_qkv_native_bhsd(x, w, None, num_heads=8, value_layout="bshd")
        strided = torch.zeros(2, 32, 512, dtype=torch.bfloat16, device=gpu_device)[:, ::2]
        assert not can_use_hip_qkv_native_bhsd(strided, w, None, num_heads=8)
        assert can_use_hip_qkv_native_bhsd(x, w, None, num_heads=8)
    # outside inference mode the strict contract refuses (as the reference's does)
    assert not can_use_hip_qkv_native_bhsd(x, w, None, num_heads=8)
