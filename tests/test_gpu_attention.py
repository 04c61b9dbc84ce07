"""GPU parity of the gfx950 causal attention kernel against the CPU oracle.

Gate (written here, applied elementwise like the official OR rule): a bf16 or
fp16 output element passes when |err| <= 2e-2 or |err| <= 1e-2 * |ref|, with
the reference computed in fp32 (float64 for the sampled long-sequence rows)
from the same 16-bit inputs.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.compare import parity_gate
from oracle.forward import causal_attention_rows, query_block_causal_attention

pytestmark = pytest.mark.gpu


def _attention_module():
    from solution.shape14 import hip_streaming_dh64

    return hip_streaming_dh64


def _inputs(batch, heads, seq, *, dtype, seed, scale_inputs=1.0):
    generator = torch.Generator().manual_seed(seed)
    shape = (batch, heads, seq, 64)
    q, k, v = (torch.randn(shape, generator=generator) * scale_inputs for _ in range(3))
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _oracle(q, k, v, scale):
    return query_block_causal_attention(q.float(), k.float(), v.float(), scale)


def _to_bsd(context_bhsd: torch.Tensor) -> torch.Tensor:
    batch, heads, seq, dim = context_bhsd.shape
    return context_bhsd.transpose(1, 2).reshape(batch, seq, heads * dim)


def _run(q, k, v, device, scale=1 / 8, **launch):
    module = _attention_module()
    with torch.inference_mode():
        output, marker = module.hip_streaming_dh64_causal_attention_bsd(
            q.to(device), k.to(device), v.to(device), scale=scale, **launch
        )
    assert marker == module.HIP_STREAMING_DH64_CAUSAL_ATTENTION_BSD_BACKEND
    torch.cuda.synchronize(device)
    return output


def _assert_parity(reference, candidate, dtype, what):
    result = parity_gate(reference, candidate.float().cpu(), dtype)
    assert result.passed, (
        f"{what}: {result.failed_elements}/{result.total_elements} failed, "
        f"max_abs={result.max_abs_error:.4g} at {result.worst_index}"
    )


# (block_m, num_warps, num_stages): 32 or 64 rows per wave, 4 or 8 waves; 3 stages = pipelined kernel
LAUNCHES = [(128, 4, 2), (256, 4, 2), (256, 8, 2), (512, 8, 2), (512, 8, 1), (128, 4, 3)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block_m,num_warps,num_stages", LAUNCHES)
@pytest.mark.parametrize(
    "batch,heads,seq",
    [(1, 1, 1), (1, 2, 17), (2, 3, 100), (2, 2, 257), (1, 2, 1000), (3, 1, 130)],
)
def test_attention_matches_oracle(gpu_device, dtype, block_m, num_warps, num_stages, batch, heads, seq):
    launch = (block_m, num_warps, num_stages)
    print(f"attention parity dtype={dtype} launch={launch} shape={(batch, heads, seq)}", flush=True)
    q, k, v = _inputs(batch, heads, seq, dtype=dtype, seed=seq * 7 + heads)
    output = _run(q, k, v, gpu_device, block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    reference = _to_bsd(_oracle(q, k, v, 1 / 8))
    _assert_parity(reference, output, dtype, f"{dtype} {block_m} {(batch, heads, seq)}")


@pytest.mark.parametrize("block_m,num_warps,num_stages", LAUNCHES)
def test_baseline_config3_attention(gpu_device, block_m, num_warps, num_stages):
    """B8 H16 S2048 Dh64, inputs N(0,1)/sqrt(64); the op
    applies the 1/sqrt(64) softmax scale on top."""

    print(f"config-3 attention launch={(block_m, num_warps, num_stages)}", flush=True)
    q, k, v = _inputs(8, 16, 2048, dtype=torch.bfloat16, seed=1234, scale_inputs=1 / 8)
    output = _run(q, k, v, gpu_device, block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    reference = _to_bsd(_oracle(q, k, v, 1 / 8))
    _assert_parity(reference, output, torch.bfloat16, "config 3")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block_m,num_warps,num_stages", [(128, 4, 3), (256, 8, 2), (512, 8, 2)])
def test_large_scores_near_one_hot_softmax(gpu_device, dtype, block_m, num_warps, num_stages):
    """Inputs scaled by 4 (scaled scores with a standard deviation of 16): the
    softmax of most rows is nearly one-hot, the running maximum rises by large
    steps and most probabilities underflow to zero.  The online rescaling
    must still match the fp32 oracle."""

    print(f"large scores {dtype} launch={(block_m, num_warps, num_stages)}", flush=True)
    q, k, v = _inputs(2, 2, 700, dtype=dtype, seed=99, scale_inputs=4.0)
    output = _run(q, k, v, gpu_device, block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    assert bool(torch.isfinite(output).all())
    reference = _to_bsd(_oracle(q, k, v, 1 / 8))
    _assert_parity(reference, output, dtype, f"large scores {dtype} {block_m}")


def test_launch_shapes_and_stages_are_bitwise_identical(gpu_device):
    """Within the double/single-buffered kernel, a query row's result does not
    depend on the tiling of the grid."""

    q, k, v = _inputs(2, 4, 777, dtype=torch.bfloat16, seed=5)
    outputs = [
        _run(q, k, v, gpu_device, block_m=block_m, num_warps=warps, num_stages=stages)
        for block_m, warps in ((128, 4), (256, 4), (256, 8), (512, 8))
        for stages in (1, 2)
    ]
    for other in outputs[1:]:
        assert torch.equal(outputs[0], other)


def test_packed_qkv_view_and_transposed_value_layouts_agree(gpu_device):
    """The reference's zero-copy split of [B,S,3D] (strided, head_dim
    contiguous V) and a seq-contiguous V^T buffer give identical results."""

    batch, seq, heads = 2, 300, 4
    width = heads * 64
    generator = torch.Generator().manual_seed(11)
    packed = torch.randn(batch, seq, 3 * width, generator=generator).to(torch.bfloat16)
    packed_gpu = packed.to(gpu_device)
    q, k, v = (
        t.transpose(1, 2) for t in packed_gpu.unflatten(-1, (3, heads, 64)).unbind(dim=2)
    )
    assert q.stride(-1) == 1 and not q.is_contiguous()
    module = _attention_module()
    with torch.inference_mode():
        from_view, _ = module.hip_streaming_dh64_causal_attention_bsd(q, k, v, scale=1 / 8)
        seq_pad = 320
        v_t = torch.zeros(batch, heads, 64, seq_pad, dtype=torch.bfloat16, device=gpu_device)
        v_t[..., :seq] = v.transpose(-1, -2)
        v_seq_major = v_t[..., :seq].transpose(-1, -2)
        assert v_seq_major.stride(-2) == 1
        from_vt, _ = module.hip_streaming_dh64_causal_attention_bsd(q, k, v_seq_major, scale=1 / 8)
    assert torch.equal(from_view, from_vt)
    reference = _to_bsd(_oracle(q.cpu(), k.cpu(), v.cpu(), 1 / 8))
    _assert_parity(reference, from_view, torch.bfloat16, "packed view")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seq,launch", [(4500, (256, 8, 2)), (1000, (256, 8, 2)), (1000, (128, 4, 2)), (1000, (128, 4, 3))])
def test_value_with_a_padded_key_stride_is_read_as_given(gpu_device, dtype, seq, launch):
    """V head_dim-contiguous with a key stride of 72 elements, its rows padded
    by 16 bytes that hold NaN: read as given (4500 keys: the scaled-key path's
    direct-to-LDS ring with a partial last tile; 1000 keys: register-staged
    tiles and the pipelined kernel), the PV operand transposed out of LDS.
    Bitwise equal to the contiguous V, finite (the padding is never read) and
    at parity with the oracle."""

    print(f"padded V key stride dtype={dtype} S={seq} launch={launch}", flush=True)
    q, k, v = _inputs(1, 3, seq, dtype=dtype, seed=seq + 7)
    padded = torch.full((1, 3, seq, 72), float("nan"), dtype=dtype)
    padded[..., :64] = v
    v_padded = padded.to(gpu_device)[..., :64]
    assert v_padded.stride(2) == 72 and v_padded.stride(3) == 1
    block_m, warps, stages = launch
    strided = _run(q, k, v_padded, gpu_device, block_m=block_m, num_warps=warps, num_stages=stages)
    contiguous = _run(q, k, v, gpu_device, block_m=block_m, num_warps=warps, num_stages=stages)
    assert bool(torch.isfinite(strided).all())
    assert torch.equal(strided, contiguous)
    reference = _to_bsd(_oracle(q, k, v, 1 / 8))
    _assert_parity(reference, strided, dtype, f"padded V key stride S={seq} launch={launch}")


@pytest.mark.parametrize("block_m,num_warps", [(256, 8), (512, 8), (128, 4)])
def test_long_sequence_value_layouts_agree_with_poisoned_padding(gpu_device, block_m, num_warps):
    """S = 16500 (scaled-key path; the last key tile is partial, and so is its
    last 8-key chunk): V as the packed head_dim-contiguous view (read as
    given) and as a caller's seq-contiguous V^T buffer whose columns past the
    sequence hold NaN (copied key-major into the workspace) give bitwise
    equal outputs, so the copy never reads a key at or past S (a NaN times
    P = 0 would show)."""

    batch, seq, heads = 1, 16_500, 2
    width = heads * 64
    print(f"value layouts S={seq} launch=({block_m}, {num_warps}, 2)", flush=True)
    generator = torch.Generator().manual_seed(29)
    packed = torch.randn(batch, seq, 3 * width, generator=generator).to(torch.bfloat16).to(gpu_device)
    q, k, v = (t.transpose(1, 2) for t in packed.unflatten(-1, (3, heads, 64)).unbind(dim=2))
    module = _attention_module()
    launch = dict(block_m=block_m, block_n=64, num_warps=num_warps, num_stages=2)
    with torch.inference_mode():
        from_view, _ = module.hip_streaming_dh64_causal_attention_bsd(q, k, v, scale=1 / 8, **launch)
        stride = seq + 12  # a multiple of 8 that leaves a partial chunk of padding after S
        v_t = torch.full((batch, heads, 64, stride), float("nan"), dtype=torch.bfloat16, device=gpu_device)
        v_t[..., :seq] = v.transpose(-1, -2)
        v_seq_major = v_t[..., :seq].transpose(-1, -2)
        assert v_seq_major.stride(-2) == 1 and v_seq_major.stride(-1) == stride
        from_vt, _ = module.hip_streaming_dh64_causal_attention_bsd(q, k, v_seq_major, scale=1 / 8, **launch)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(from_view).all())
    assert torch.equal(from_view, from_vt)


def test_constant_value_rows_are_reproduced(gpu_device):
    """Softmax weights sum to one, so a constant V column yields that constant."""

    q, k, _ = _inputs(1, 2, 513, dtype=torch.bfloat16, seed=3)
    columns = torch.linspace(-3, 3, 64).to(torch.bfloat16)
    v = columns.expand(1, 2, 513, 64).contiguous()
    output = _run(q, k, v, gpu_device).float().cpu()
    expected = columns.float().repeat(2).expand(1, 513, 128)
    assert (output - expected).abs().max().item() <= 2e-2


def test_zero_query_gives_running_prefix_mean(gpu_device):
    """Q = 0 makes every visible key equally likely: row i is mean(V[0..i])."""

    _, k, v = _inputs(1, 1, 300, dtype=torch.bfloat16, seed=9)
    q = torch.zeros_like(k)
    output = _run(q, k, v, gpu_device).float().cpu()[0]
    prefix = torch.cumsum(v[0, 0].double(), dim=0) / torch.arange(1, 301).double()[:, None]
    _assert_parity(prefix.float(), output, torch.bfloat16, "prefix mean")


def test_first_row_copies_first_value(gpu_device):
    q, k, v = _inputs(2, 3, 64, dtype=torch.bfloat16, seed=21)
    output = _run(q, k, v, gpu_device).cpu()
    for head in range(3):
        assert torch.equal(output[:, 0, head * 64 : (head + 1) * 64], v[:, head, 0])


@pytest.mark.parametrize("block_m,num_warps,num_stages", [(256, 8, 2), (128, 4, 2), (128, 4, 3)])
@pytest.mark.parametrize("batch,heads,seq", [(5, 16, 8192), (3, 8, 2048), (1, 12, 4096)])
def test_issue_order_covers_every_tile(gpu_device, block_m, num_warps, num_stages, batch, heads, seq):
    """Every (batch*head, query tile) workgroup runs exactly once under the
    grouped issue order, including several head groups with a smaller last
    one (B5 H16 S8192: 10 heads per XCD) and the fallback order when
    batch*heads is not a multiple of 8 (B1 H12).

    V is constant per head (a multiple of 1/16, exact in bf16), so every
    output row of head bh equals that constant: the softmax weights sum to
    one and the fp32 accumulation error (below 1e-3 relative) is under half
    a bf16 ulp.  Two calls with different constants make a tile that was
    never written show the previous call's value."""

    launch = dict(block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    print(f"issue order launch={launch} shape={(batch, heads, seq)}", flush=True)
    module = _attention_module()
    generator = torch.Generator(device=gpu_device).manual_seed(seq + heads)
    shape = (batch, heads, seq, 64)
    q, k = (
        (torch.randn(shape, generator=generator, device=gpu_device) / 8).to(torch.bfloat16)
        for _ in range(2)
    )
    index = torch.arange(batch * heads, device=gpu_device).reshape(batch, heads)
    for sign in (1.0, -1.0):
        constants = (sign * ((index % 15) + 1) / 16).to(torch.bfloat16)
        v = constants[:, :, None, None].expand(shape).contiguous()
        with torch.inference_mode():
            output, _ = module.hip_streaming_dh64_causal_attention_bsd(q, k, v, scale=1 / 8, **launch)
        expected = constants[:, None, :, None].expand(batch, seq, heads, 64).reshape(batch, seq, heads * 64)
        torch.cuda.synchronize(gpu_device)
        mismatched = (output != expected).sum().item()
        assert mismatched == 0, f"{mismatched} elements differ from their head's constant (sign {sign})"


@pytest.mark.parametrize("block_m,num_warps,num_stages", LAUNCHES)
def test_batch_slices_are_independent(gpu_device, block_m, num_warps, num_stages):
    """Running a sub-batch gives bitwise the rows of the full batch (the
    property the streamed chunk driver relies on)."""

    launch = dict(block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    q, k, v = _inputs(4, 2, 400, dtype=torch.bfloat16, seed=17)
    full = _run(q, k, v, gpu_device, **launch)
    part = _run(q[1:3], k[1:3], v[1:3], gpu_device, **launch)
    assert torch.equal(full[1:3], part)


@pytest.mark.parametrize("block_m,num_warps,num_stages", [(128, 4, 3), (256, 4, 2), (512, 8, 2)])
def test_long_sequence_sampled_rows(gpu_device, block_m, num_warps, num_stages):
    """S = 100000 (the long-sequence configuration's length): sampled rows,
    including the last ones that see every key, against float64 per-row math."""

    seq = 100_000
    print(f"long-sequence attention S=100000 launch={(block_m, num_warps, num_stages)}", flush=True)
    q, k, v = _inputs(1, 2, seq, dtype=torch.bfloat16, seed=2024)
    output = _run(
        q, k, v, gpu_device, block_m=block_m, num_warps=num_warps, num_stages=num_stages
    ).float().cpu()
    rng = np.random.default_rng(0)
    rows = np.unique(
        np.concatenate([np.arange(0, 40), np.arange(seq - 40, seq), rng.integers(0, seq, 40)])
    )
    for head in range(2):
        expected = causal_attention_rows(
            q[0, head].float().numpy(), k[0, head].float().numpy(), v[0, head].float().numpy(),
            rows, 1 / 8,
        )
        actual = output[0, rows, head * 64 : (head + 1) * 64]
        _assert_parity(torch.from_numpy(expected).float(), actual, torch.bfloat16, f"head {head}")


@pytest.mark.parametrize("case", ["large_scores", "late_outlier_key"])
def test_score_bound_path_sampled_rows(gpu_device, case):
    """S = 20000 runs with the key-norm pre-pass, where rows whose score
    bound c |q| max|k| stays within 2^64 of their shift skip the tile maximum.
    Large scores (inputs x4) keep the bound above that margin, so every tile
    forms its maximum; a single late key with a 40x norm makes the bound of
    its tile jump, and the rows that see it must raise their shift there.
    Sampled rows against float64 per-row math."""

    seq = 20_000
    print(f"score-bound attention S={seq} case={case}", flush=True)
    scale = 4.0 if case == "large_scores" else 1.0
    q, k, v = _inputs(1, 2, seq, dtype=torch.bfloat16, seed=77, scale_inputs=scale)
    if case == "late_outlier_key":
        k[0, :, 15000] = (k[0, :, 15000].float() * 40).to(torch.bfloat16)
    outputs = [
        _run(q, k, v, gpu_device, block_m=block_m, num_warps=warps, num_stages=2).float().cpu()
        for block_m, warps in ((256, 8), (128, 4))
    ]
    assert torch.equal(outputs[0], outputs[1])
    assert bool(torch.isfinite(outputs[0]).all())
    rng = np.random.default_rng(1)
    rows = np.unique(np.concatenate([
        np.arange(0, 20), np.arange(14990, 15030), np.arange(seq - 20, seq), rng.integers(0, seq, 40)
    ]))
    for head in range(2):
        expected = causal_attention_rows(
            q[0, head].float().numpy(), k[0, head].float().numpy(), v[0, head].float().numpy(),
            rows, 1 / 8,
        )
        actual = outputs[0][0, rows, head * 64 : (head + 1) * 64]
        _assert_parity(torch.from_numpy(expected).float(), actual, torch.bfloat16, f"{case} head {head}")


def test_fp16_score_bound_keeps_probabilities_in_range(gpu_device):
    """fp16 P overflows above 65504: on the score-bound path (S >= 4096) an
    fp16 row may skip its tile maximum only while its bound keeps every
    probability below 2^15.  Key 15000 is set to 3.8 x query 15005, so that
    row's score for it is about 40 powers of two above its shift while the
    tile's bound stays within 2^64 of the shift: bf16 P could skip the
    maximum there, fp16 P must not (2^40 would be inf)."""

    seq = 20_000
    print(f"fp16 score-bound attention S={seq}", flush=True)
    q, k, v = _inputs(1, 2, seq, dtype=torch.float16, seed=5)
    k[0, :, 15000] = (q[0, :, 15005].float() * 3.8).to(torch.float16)
    output = _run(q, k, v, gpu_device, block_m=256, num_warps=8, num_stages=2).float().cpu()
    assert bool(torch.isfinite(output).all())
    rng = np.random.default_rng(2)
    rows = np.unique(np.concatenate([
        np.arange(0, 10), np.arange(14998, 15012), np.arange(seq - 10, seq), rng.integers(0, seq, 40)
    ]))
    for head in range(2):
        expected = causal_attention_rows(
            q[0, head].float().numpy(), k[0, head].float().numpy(), v[0, head].float().numpy(),
            rows, 1 / 8,
        )
        actual = output[0, rows, head * 64 : (head + 1) * 64]
        _assert_parity(torch.from_numpy(expected).float(), actual, torch.float16, f"fp16 head {head}")


@pytest.mark.parametrize("dtype,magnitude", [(torch.bfloat16, 1.0), (torch.float16, 0.5)])
def test_scaled_key_path_sampled_rows(gpu_device, dtype, magnitude):
    """S = 20000 with moderate scores: every workgroup's bound c |q| max|k|
    is within the scaled-key limit (32 for bf16 P, 15 for fp16 P), so the
    scores come from the fp16 MFMA on the pre-pass's scaled keys and P =
    exp2(score) without a shift.  Sampled rows against float64 per-row math,
    and the 8-wave and 4-wave launches bitwise equal."""

    seq = 20_000
    print(f"scaled-key attention S={seq} {dtype} x{magnitude}", flush=True)
    q, k, v = _inputs(1, 2, seq, dtype=dtype, seed=91, scale_inputs=magnitude)
    outputs = [
        _run(q, k, v, gpu_device, block_m=block_m, num_warps=warps, num_stages=2).float().cpu()
        for block_m, warps in ((256, 8), (128, 4))
    ]
    assert torch.equal(outputs[0], outputs[1])
    rng = np.random.default_rng(3)
    rows = np.unique(np.concatenate([np.arange(0, 20), np.arange(seq - 20, seq), rng.integers(0, seq, 60)]))
    for head in range(2):
        expected = causal_attention_rows(
            q[0, head].float().numpy(), k[0, head].float().numpy(), v[0, head].float().numpy(),
            rows, 1 / 8,
        )
        actual = outputs[0][0, rows, head * 64 : (head + 1) * 64]
        _assert_parity(torch.from_numpy(expected).float(), actual, dtype, f"scaled keys head {head}")


@pytest.mark.parametrize("dtype,bound,limit", [(torch.bfloat16, 31.0, 32.0), (torch.float16, 14.5, 15.0)])
@pytest.mark.parametrize("value_scale", [1.0, 4.0])
def test_scaled_key_path_near_its_bound_with_aligned_rows(gpu_device, dtype, bound, limit, value_scale):
    """Queries and keys that share one direction (q nearly parallel to many
    keys), scaled so that c max|q| max|k| sits just under the scaled-key limit
    (32 for bf16 P, 15 for fp16 P): every 512-row block takes the scaled-key
    path with scores close to the limit, where the fp16 rounding of c k
    (unit roundoff 2^-11) weighs most.  Sampled rows against float64 per-row
    math: with V of magnitude 1 at the gate; with V of magnitude 4, where
    rounding P to 16 bits before PV (the reference's order) alone moves a
    near-one-hot row by more than 2e-2, no less accurate than the official
    order in the same dtype (scores, softmax cast and PV as
    official/torch_transformer_benchmark.py:97-112)."""

    seq, heads = 4608, 2
    c = 0.125 * math.log2(math.e)
    generator = torch.Generator().manual_seed(17)
    direction = torch.randn(64, generator=generator)
    direction /= direction.norm()

    def aligned():
        noise = torch.randn(1, heads, seq, 64, generator=generator) * 0.5
        along = torch.randn(1, heads, seq, 1, generator=generator) * 3.0
        return noise + along * direction

    k = aligned().to(dtype)
    q = aligned()
    factor = bound / (c * q.norm(dim=-1).max() * k.float().norm(dim=-1).max())
    q = (q * factor).to(dtype)
    reach = c * q.float().norm(dim=-1).max() * k.float().norm(dim=-1).max()
    # within the scaled-key limit (the 16-bit rounding of q moves it a little)
    assert bound - 1.0 < float(reach) < limit, float(reach)
    v = (torch.randn(1, heads, seq, 64, generator=generator) * value_scale).to(dtype)
    print(f"scaled-key bound {dtype} reach={float(reach):.2f} |v|x{value_scale}", flush=True)
    output = _run(q, k, v, gpu_device, block_m=256, num_warps=8, num_stages=2).float().cpu()
    official = _to_bsd(query_block_causal_attention(q, k, v, 1 / 8)).float()
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([np.arange(0, 8), np.arange(seq - 8, seq), rng.integers(0, seq, 48)]))
    for head in range(heads):
        expected = torch.from_numpy(causal_attention_rows(
            q[0, head].float().numpy(), k[0, head].float().numpy(), v[0, head].float().numpy(), rows, 1 / 8
        )).float()
        columns = slice(head * 64, (head + 1) * 64)
        result = parity_gate(expected, output[0, rows, columns], dtype)
        order = parity_gate(expected, official[0, rows, columns], dtype)
        print(f"  head {head}: HIP max_abs={result.max_abs_error:.3g} failed={result.failed_elements}; "
              f"official order max_abs={order.max_abs_error:.3g} failed={order.failed_elements}", flush=True)
        if value_scale == 1.0:
            _assert_parity(expected, output[0, rows, columns], dtype, f"aligned rows head {head}")
        else:
            assert result.failed_elements <= order.failed_elements + 1, (result, order)
            assert result.max_abs_error <= max(2e-2, 1.25 * order.max_abs_error), (result, order)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seq", [4095, 4096, 4097])
def test_preparation_threshold_boundary(gpu_device, dtype, seq):
    """4095 keys run the shifted path, 4096 and more the preparation launch
    and the scaled-key path (with V in [B, H, S, 64] the workspace holds
    only the norm tables and scaled keys, and only then).  Every row on both sides of the
    boundary against the fp32 oracle, under the 8-wave ring launch and a
    4-wave launch."""

    from solution.kernels.hip import _library

    library = _library.load_library()
    code = 1 if dtype == torch.float16 else 2
    workspace = library.sah_causal_attention_workspace_bytes(1, 2, seq, 64, 64, 1, code)
    assert (workspace > 0) == (seq >= 4096), (seq, workspace)
    q, k, v = _inputs(1, 2, seq, dtype=dtype, seed=seq)
    reference = _to_bsd(_oracle(q, k, v, 1 / 8))
    for block_m, warps in ((256, 8), (128, 4)):
        print(f"threshold boundary dtype={dtype} S={seq} launch=({block_m}, {warps}, 2)", flush=True)
        output = _run(q, k, v, gpu_device, block_m=block_m, num_warps=warps, num_stages=2)
        _assert_parity(reference, output, dtype, f"S={seq} launch ({block_m}, {warps})")


def test_scaled_keys_in_the_workspace(gpu_device):
    """The preparation launch writes the largest |k| of every 64-key tile,
    then the largest |k| and the largest |q| of every 512-row block, then
    every key times c = scale * log2(e) rounded to fp16 as [batch*heads]
    [key_tiles * 64][64].  Norms are checked against float64 norms of the
    same rows (fp32 sums of squares: within a few ulps), the blocks against
    the tiles' own maxima (bitwise: the same fp32 values, maximized), the
    scaled keys bitwise against fp32 products rounded to fp16."""

    from solution.kernels.hip._library import load_library

    batch, heads, seq = 1, 3, 16_500
    q, k, v = _inputs(batch, heads, seq, dtype=torch.bfloat16, seed=12)
    # one row of each of Q and K in the last block far above the rest, so a
    # block maximum taken over the wrong rows shows
    k[0, 1, 16_400] *= 5
    q[0, 2, 16_499] *= 7
    library = load_library()
    qd, kd, value = q.to(gpu_device), k.to(gpu_device), v.to(gpu_device)
    need = library.sah_causal_attention_workspace_bytes(batch, heads, seq, 64, value.stride(2), 1, 2)
    tiles = -(-seq // 64)
    row_blocks = -(-seq // 512)
    table = -(-(batch * heads * tiles * 4) // 256) * 256
    block_bytes = -(-(2 * batch * heads * row_blocks * 4) // 256) * 256
    assert need == table + block_bytes + batch * heads * tiles * 64 * 64 * 2
    workspace = torch.zeros(need, dtype=torch.uint8, device=gpu_device)
    out = torch.empty(batch, seq, heads * 64, dtype=torch.bfloat16, device=gpu_device)
    scale = 0.125
    status = library.sah_causal_attention_bsd(
        qd.data_ptr(), kd.data_ptr(), value.data_ptr(), out.data_ptr(), batch, heads, seq, 64,
        *qd.stride()[:3], *kd.stride()[:3], *value.stride(), out.stride(0), out.stride(1),
        scale, 2, 256, 64, 8, 2, workspace.data_ptr(), need, torch.cuda.current_stream().cuda_stream,
    )
    assert status == 0
    torch.cuda.synchronize()
    host = workspace.cpu()

    def row_norms(x):
        padded = torch.zeros(batch * heads, row_blocks * 512, 64, dtype=torch.float64)
        padded[:, :seq] = x.double().reshape(batch * heads, seq, 64)
        return padded.norm(dim=-1)

    knorm64, qnorm64 = row_norms(k), row_norms(q)
    norms = host[: batch * heads * tiles * 4].view(torch.float32).view(batch * heads, tiles)
    want_norms = knorm64[:, : tiles * 64].view(batch * heads, tiles, 64).amax(-1)
    assert torch.allclose(norms.double(), want_norms, rtol=1e-5, atol=0)
    start = table
    kblock = host[start : start + batch * heads * row_blocks * 4].view(torch.float32).view(batch * heads, row_blocks)
    start += batch * heads * row_blocks * 4
    qblock = host[start : start + batch * heads * row_blocks * 4].view(torch.float32).view(batch * heads, row_blocks)
    per_block = norms.new_zeros(batch * heads, row_blocks * 8)
    per_block[:, :tiles] = norms
    assert torch.equal(kblock, per_block.view(batch * heads, row_blocks, 8).amax(-1))
    assert torch.allclose(kblock.double(), knorm64.view(batch * heads, row_blocks, 512).amax(-1), rtol=1e-5, atol=0)
    assert torch.allclose(qblock.double(), qnorm64.view(batch * heads, row_blocks, 512).amax(-1), rtol=1e-5, atol=0)
    assert int(kblock[1].argmax()) == row_blocks - 1 and int(qblock[2].argmax()) == row_blocks - 1
    scaled = host[table + block_bytes :].view(torch.float16).view(batch * heads, tiles * 64, 64)[:, :seq]
    want = (k.float().reshape(batch * heads, seq, 64) * np.float32(scale * math.log2(math.e))).half()
    assert torch.equal(scaled, want)


def test_invalid_launch_and_ineligible_inputs_raise(gpu_device):
    module = _attention_module()
    q, k, v = (t.to(gpu_device) for t in _inputs(1, 1, 64, dtype=torch.bfloat16, seed=1))
    with torch.inference_mode():
        with pytest.raises(ValueError):
            module.prevalidated_hip_streaming_dh64_causal_attention_bsd(q, k, v, block_m=64)
        # mixed dtypes, and fp32 with a seq-contiguous V (the fp32 kernel reads
        # V head_dim-contiguous), are ineligible
        with pytest.raises(RuntimeError, match="ineligible"):
            module.hip_streaming_dh64_causal_attention_bsd(q.float(), k, v)
        vt = v.float().transpose(-2, -1).contiguous().transpose(-2, -1)
        with pytest.raises(RuntimeError, match="ineligible"):
            module.hip_streaming_dh64_causal_attention_bsd(q.float(), k.float(), vt)
    assert not module.can_use_hip_streaming_dh64_causal_attention(q, k, v, causal=False)


SCALE_LAUNCHES = [(128, 4, 2), (256, 8, 2), (512, 8, 1), (128, 4, 3)]


@pytest.mark.parametrize("block_m,num_warps,num_stages", SCALE_LAUNCHES)
@pytest.mark.parametrize("seq", [300, 16500])
def test_zero_scale_is_the_prefix_mean(gpu_device, block_m, num_warps, num_stages, seq):
    """softmax(0 * s + causal mask) weighs every visible key equally: row i is
    the mean of V[0..i], whatever Q and K hold (the reference scales the
    scores before its running maximum, so it is defined for any scale).
    S = 16500 also runs the key-norm score bound."""

    launch = (block_m, num_warps, num_stages)
    print(f"zero scale launch={launch} seq={seq}", flush=True)
    q, k, v = _inputs(1, 2, seq, dtype=torch.bfloat16, seed=seq + 3, scale_inputs=3.0)
    output = _run(q, k, v, gpu_device, scale=0.0, block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    prefix = v.double().cumsum(dim=2) / torch.arange(1, seq + 1, dtype=torch.float64).view(1, 1, seq, 1)
    _assert_parity(_to_bsd(prefix.float()), output, torch.bfloat16, f"zero scale {launch}")


@pytest.mark.parametrize("block_m,num_warps,num_stages", SCALE_LAUNCHES)
@pytest.mark.parametrize("scale", [-1 / 8, -0.4])
def test_negative_scale_matches_oracle_and_negated_query(gpu_device, block_m, num_warps, num_stages, scale):
    """A negative scale is the oracle's softmax of scale * q.k, and bitwise the
    positive scale on the negated query."""

    launch = dict(block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    print(f"negative scale {scale} launch={launch}", flush=True)
    q, k, v = _inputs(2, 2, 333, dtype=torch.bfloat16, seed=17)
    output = _run(q, k, v, gpu_device, scale=scale, **launch)
    assert bool(torch.isfinite(output).all())
    _assert_parity(_to_bsd(_oracle(q, k, v, scale)), output, torch.bfloat16, f"scale {scale}")
    flipped = _run(-q, k, v, gpu_device, scale=-scale, **launch)
    assert torch.equal(output, flipped)


def test_negative_scale_on_the_scaled_key_path(gpu_device):
    """S = 16500 (key-norm pre-pass, scaled keys): a negative scale folds its
    sign into the query, so it equals the positive scale on the negated query
    bitwise, and sampled rows match float64."""

    seq = 16_500
    print(f"negative scale scaled-key path S={seq}", flush=True)
    q, k, v = _inputs(1, 2, seq, dtype=torch.bfloat16, seed=23)
    launch = dict(block_m=256, num_warps=8, num_stages=2)
    output = _run(q, k, v, gpu_device, scale=-1 / 8, **launch)
    flipped = _run(-q, k, v, gpu_device, scale=1 / 8, **launch)
    assert torch.equal(output, flipped)
    rows = np.unique(np.concatenate([np.arange(0, 10), np.arange(seq - 10, seq), np.arange(8000, 8040)]))
    for head in range(2):
        expected = causal_attention_rows(
            q[0, head].float().numpy(), k[0, head].float().numpy(), v[0, head].float().numpy(),
            rows, -1 / 8,
        )
        actual = output.float().cpu()[0, rows, head * 64 : (head + 1) * 64]
        _assert_parity(torch.from_numpy(expected).float(), actual, torch.bfloat16, f"negative scale head {head}")


@pytest.mark.parametrize("block_m,num_warps,num_stages", [(128, 4, 2), (256, 8, 2)])
@pytest.mark.parametrize(
    "batch,heads,seq",
    [(1, 1, 1), (1, 2, 17), (2, 3, 100), (2, 2, 257), (1, 2, 1000), (3, 1, 130), (2, 4, 128)],
)
def test_fp32_attention_matches_oracle_at_1e4(gpu_device, block_m, num_warps, num_stages, batch, heads, seq):
    """fp32 inputs: the fp32 kernel (scores, softmax and PV in fp32, P not
    rounded) against the oracle's fp32 query-block order, at the fp32 gate
    |err| <= 1e-4 or |err| <= 1e-4 |ref|."""

    print(f"fp32 attention launch={(block_m, num_warps, num_stages)} shape={(batch, heads, seq)}", flush=True)
    q, k, v = _inputs(batch, heads, seq, dtype=torch.float32, seed=seq * 5 + heads)
    output = _run(q, k, v, gpu_device, block_m=block_m, num_warps=num_warps, num_stages=num_stages)
    assert output.dtype == torch.float32
    reference = _to_bsd(_oracle(q, k, v, 1 / 8))
    _assert_parity(reference, output, torch.float32, f"fp32 {(batch, heads, seq)}")


@pytest.mark.parametrize("scale", [0.0, -0.125])
def test_fp32_attention_scale_sign_and_packed_views(gpu_device, scale):
    """fp32 through packed-QKV views (row stride 3D), with a zero and a
    negative scale."""

    batch, heads, seq = 2, 4, 300
    generator = torch.Generator().manual_seed(11)
    packed = torch.randn(batch, seq, 3 * heads * 64, generator=generator)
    q, k, v = (packed[..., i * heads * 64 : (i + 1) * heads * 64].view(batch, seq, heads, 64).transpose(1, 2)
               for i in range(3))
    module = _attention_module()
    device_packed = packed.to(gpu_device)
    dq, dk, dv = (device_packed[..., i * heads * 64 : (i + 1) * heads * 64].view(batch, seq, heads, 64).transpose(1, 2)
                  for i in range(3))
    with torch.inference_mode():
        output, _ = module.hip_streaming_dh64_causal_attention_bsd(dq, dk, dv, scale=scale)
    torch.cuda.synchronize(gpu_device)
    reference = _to_bsd(_oracle(q, k, v, scale))
    _assert_parity(reference, output, torch.float32, f"fp32 packed scale {scale}")
