"""Pins of the CPU oracle (runs without a GPU).

Each oracle function is checked against something that does not share its
code: float64 library routines, scalar-loop brute force, the reference's own
known answers, or invariants a plausible mistake would break.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import norm as oracle_norm
from oracle.compare import OFFICIAL_ATOL, OFFICIAL_RTOL, official_compare, parity_gate
from oracle.forward import (
    TransformerConfig,
    causal_attention_rows,
    default_init_weights,
    dense_causal_attention,
    forward,
    generate_input,
    query_block_causal_attention,
    query_block_rows,
    xavier_init_weights,
)
from oracle.workload import (
    C3_ATTENTION,
    C3_NORM,
    C5,
    causal_attention_flops,
    estimated_model_flops,
    residual_norm_bytes,
)

GOLDEN = Path(__file__).resolve().parent / "golden"
C1 = TransformerConfig(2, 128, 256, 4, 1024, 2, True)


def test_c1_forward_matches_float64_library_golden():
    """Official op order in fp32 vs float64 SDPA/layer_norm/gelu (config 1)."""

    golden = np.load(GOLDEN / "c1_forward.npz")
    state = default_init_weights(C1, seed=1234)
    sums = np.array([float(state[name].double().sum()) for name in golden["weight_names"]])
    np.testing.assert_allclose(sums, golden["weight_sums"], rtol=0, atol=1e-9)
    x = generate_input(C1, seed=1234)
    assert np.array_equal(x.numpy(), golden["x"])
    out = forward(state, x, C1)
    result = parity_gate(torch.from_numpy(golden["out"]), out, torch.float32)
    assert result.passed, result
    assert result.max_abs_error < 2e-5


def test_dense_attention_matches_scalar_loop_golden():
    golden = np.load(GOLDEN / "tiny_attention.npz")
    q, k, v = (torch.from_numpy(golden[name]) for name in ("q", "k", "v"))
    out = dense_causal_attention(q, k, v, 1 / math.sqrt(4))
    # the official order runs the softmax in fp32 even for float64 scores
    np.testing.assert_allclose(out.numpy(), golden["out"], rtol=2e-6, atol=2e-6)


def test_query_block_order_equals_dense_order():
    """Restates the reference's check that the query-block path keeps the
    official operation order (tests/solution/test_causal_operators.py:62-84)."""

    generator = torch.Generator().manual_seed(19)
    q, k, v = (torch.randn(2, 2, 300, 16, generator=generator) for _ in range(3))
    dense = dense_causal_attention(q, k, v, 0.25)
    for block in (1, 7, 128, 300, 512):
        torch.testing.assert_close(query_block_causal_attention(q, k, v, 0.25, query_block=block), dense)
    # one block anywhere in the sequence (the CPU baseline times sampled blocks)
    torch.testing.assert_close(query_block_rows(q, k, v, 0.25, 37, 101), dense[..., 37:101, :])
    torch.testing.assert_close(query_block_rows(q, k, v, 0.25, 299, 300), dense[..., 299:, :])


def test_attention_matches_torch_sdpa_float64():
    generator = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 3, 50, 64, generator=generator, dtype=torch.float64) for _ in range(3))
    expected = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.125)
    # fp32 softmax inside the official order bounds the agreement at fp32 level
    torch.testing.assert_close(dense_causal_attention(q, k, v, 0.125), expected, rtol=1e-6, atol=1e-6)


def test_attention_rows_match_dense_float64():
    generator = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(1, 1, 200, 64, generator=generator, dtype=torch.float64) for _ in range(3))
    dense = dense_causal_attention(q, k, v, 0.125)[0, 0].numpy()
    rows = np.array([0, 1, 99, 199])
    got = causal_attention_rows(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), rows, 0.125)
    np.testing.assert_allclose(got, dense[rows], rtol=1e-6, atol=1e-6)
    exact = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.125)[0, 0].numpy()
    np.testing.assert_allclose(got, exact[rows], rtol=1e-12, atol=1e-12)


def test_attention_mask_side_and_first_row():
    """Row 0 sees only key 0; a mistake on the mask side changes both checks."""

    generator = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 1, 10, 8, generator=generator, dtype=torch.float64) for _ in range(3))
    out = dense_causal_attention(q, k, v, 1.0)
    torch.testing.assert_close(out[0, 0, 0], v[0, 0, 0])
    k2 = k.clone()
    k2[0, 0, 9] += 100.0  # change the last key: every row before it is unaffected
    v2 = v.clone()
    v2[0, 0, 9] -= 50.0
    out2 = dense_causal_attention(q, k2, v2, 1.0)
    torch.testing.assert_close(out2[0, 0, :9], out[0, 0, :9])
    assert not torch.allclose(out2[0, 0, 9], out[0, 0, 9])


def test_layer_norm_matches_scalar_loop_golden_and_library():
    golden = np.load(GOLDEN / "tiny_layer_norm.npz")
    value, update, weight, bias = (torch.from_numpy(golden[n]) for n in ("value", "update", "weight", "bias"))
    residual, normalized = oracle_norm.residual_layer_norm(value, update, weight, bias)
    np.testing.assert_allclose(normalized.numpy(), golden["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(residual.numpy(), golden["value"] + golden["update"], rtol=0, atol=0)
    library = F.layer_norm(value + update, (8,), weight, bias, 1e-5)
    torch.testing.assert_close(normalized, library)
    row = oracle_norm.layer_norm_loop(golden["value"][1] + golden["update"][1], golden["weight"], golden["bias"], 1e-5)
    np.testing.assert_allclose(row, golden["out"][1], rtol=1e-12, atol=1e-12)


def test_residual_is_rounded_to_the_stream_dtype_before_normalizing():
    value = torch.tensor([[1.0, 2.0, 3.0, 4.0]], dtype=torch.bfloat16)
    update = torch.tensor([[1e-3, -1e-3, 1e-3, 0.0]], dtype=torch.bfloat16)
    residual, normalized = oracle_norm.residual_layer_norm(value, update, None, None)
    assert residual.dtype == torch.bfloat16
    assert torch.equal(residual, (value.double() + update.double()).to(torch.bfloat16))
    expected = oracle_norm.layer_norm(residual, None, None)
    assert torch.equal(normalized, expected)


def test_rms_norm_matches_library():
    generator = torch.Generator().manual_seed(6)
    x = torch.randn(5, 32, generator=generator, dtype=torch.float64)
    w = torch.randn(32, generator=generator, dtype=torch.float64)
    torch.testing.assert_close(oracle_norm.rms_norm(x, w, 1e-6), F.rms_norm(x, (32,), w, 1e-6))


def test_constant_row_normalizes_to_bias():
    x = torch.full((2, 16), 3.0, dtype=torch.float64)
    b = torch.arange(16, dtype=torch.float64)
    assert torch.equal(oracle_norm.layer_norm(x, torch.ones(16, dtype=torch.float64), b), b.expand(2, 16))


def test_official_comparator_is_an_or_rule():
    reference = torch.tensor([1.0, 100.0, 0.0, 1.0])
    candidate = torch.tensor([1.0015, 101.5, 0.0019, float("nan")])
    result = official_compare(reference, candidate, rtol=OFFICIAL_RTOL, atol=OFFICIAL_ATOL)
    # 1.0015: abs ok; 101.5: rel 1.5% ok; 0.0019: abs ok; nan fails.
    assert result.failed_elements == 1
    strict = official_compare(reference[:3], candidate[:3], rtol=0.01, atol=0.001)
    assert strict.failed_elements == 2  # 101.5 (1.5%) and 0.0019 fail; 1.0015 passes on rel
    # |err| = 0.021 at ref 1: fails the OR rule although atol + rtol*|ref| = 0.022 would pass.
    summed = official_compare(torch.tensor([1.0]), torch.tensor([1.021]), rtol=0.02, atol=0.002)
    assert not summed.passed
    assert OFFICIAL_RTOL == 0.02 and OFFICIAL_ATOL == 0.002


def test_flop_models_reproduce_reference_known_answers():
    # tests/benchmarking/test_shape14_measure.py:45-48 of the reference
    assert estimated_model_flops(batch=8, seq=16, width=32, ffn=32, layers=2) == 3_407_872
    # final_performance.json:421 of the reference (official Shape 14, F=1024)
    assert estimated_model_flops(batch=32, seq=100000, width=1024, ffn=1024, layers=2) == 1_391_250_636_800_000
    b, h, s, d = C3_ATTENTION
    assert causal_attention_flops(b, h, s, d) == 68_753_031_168
    assert causal_attention_flops(2, 16, 100000, 64) * 16 * C5.num_layers == 1_310_733_107_200_000
    # brute force on a tiny causal triangle: QK^T and PV each 2*Dh per pair
    pairs = sum(i + 1 for i in range(5))
    assert causal_attention_flops(1, 1, 5, 3) == 4 * 3 * pairs
    rows, width = C3_NORM
    assert residual_norm_bytes(rows, width, params=0) == 134_217_728


def test_seeded_inputs_follow_the_official_generator():
    config = TransformerConfig(2, 3, 4, 2, 8, 1, True)
    generator = torch.Generator().manual_seed(99)
    expected = torch.randn(2, 3, 4, generator=generator) * 0.5
    assert torch.equal(generate_input(config, 99, input_scale=0.5), expected)


def test_default_init_follows_linear_init_bounds():
    state = default_init_weights(TransformerConfig(1, 4, 64, 4, 128, 1, True), seed=0)
    bound = 1 / math.sqrt(64)
    assert state["layers.0.attention.q_proj.weight"].abs().max() <= bound
    assert state["layers.0.ffn_out.weight"].abs().max() <= 1 / math.sqrt(128)
    assert torch.equal(state["layers.0.norm1.weight"], torch.ones(64))
    assert torch.equal(state["final_norm.bias"], torch.zeros(64))


def test_xavier_init_bounds_and_zero_biases():
    config = TransformerConfig(1, 4, 64, 4, 256, 2, True)
    state = xavier_init_weights(config, seed=1)
    bound = math.sqrt(6 / (64 + 256))
    weight = state["layers.1.ffn_in.weight"]
    assert weight.shape == (256, 64) and weight.abs().max() <= bound
    assert weight.abs().max() > 0.9 * bound
    assert torch.equal(state["layers.0.attention.out_proj.bias"], torch.zeros(64))
    assert torch.equal(xavier_init_weights(config, seed=1)["layers.0.attention.q_proj.weight"],
                       state["layers.0.attention.q_proj.weight"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_forward_prefix_is_causal(dtype):
    """Rows before t do not depend on tokens at or after t (the property the
    long-sequence GPU test uses to check a 100k-token forward on a prefix)."""

    config = TransformerConfig(1, 40, 64, 4, 128, 2, True)
    state = default_init_weights(config, seed=3)
    x = generate_input(config, 3).to(dtype)
    full = forward(state, x, config)
    prefix = forward(state, x[:, :25], TransformerConfig(1, 25, 64, 4, 128, 2, True))
    assert torch.equal(full[:, :25], prefix)


# ---------------------------------------------------------------------------
# The model-level accuracy rule (autotune.accuracy), shared by the launch
# search's publication gate and oracle.compare.model_parity.


def _summary(max_abs=0.1, mean_abs=0.01, outside=100, total=1_000_000, finite=True):
    from autotune.accuracy import ErrorSummary

    return ErrorSummary(max_abs, mean_abs, outside, total, finite)


def test_accuracy_rule_bounds_each_statistic_at_its_own_limit():
    from autotune.accuracy import summary_no_less_accurate as ok

    incumbent = _summary()
    assert ok(incumbent, incumbent)
    # max-abs: within 1.25x of the incumbent's (a wrong factor or a flipped
    # inequality moves one of these two)
    assert ok(_summary(max_abs=0.1249), incumbent)
    assert not ok(_summary(max_abs=0.1251), incumbent)
    # ... or within the 2e-2 gate when the incumbent is more accurate than that
    tiny = _summary(max_abs=0.001)
    assert ok(_summary(max_abs=0.0199), tiny)
    assert not ok(_summary(max_abs=0.0201), tiny)
    # mean-abs: 1.25x + 1e-4
    assert ok(_summary(mean_abs=0.01259), incumbent)
    assert not ok(_summary(mean_abs=0.01261), incumbent)
    # elements outside the gate: 1.25x + 1e-4 of the elements (125 + 100)
    assert ok(_summary(outside=225), incumbent)
    assert not ok(_summary(outside=226), incumbent)
    # a non-finite candidate never passes, whatever its statistics
    assert not ok(_summary(finite=False), incumbent)
    # the roles are not symmetric: a worse candidate fails against a better incumbent
    assert ok(_summary(max_abs=0.05, mean_abs=0.005, outside=10), incumbent)
    assert not ok(incumbent, _summary(max_abs=0.05, mean_abs=0.005, outside=10))
    with pytest.raises(ValueError):
        ok(_summary(total=10), incumbent)


def test_error_summary_applies_the_or_gate_and_flags_non_finite():
    from autotune.accuracy import summarize_errors

    reference = torch.tensor([1.0, 5.0, -5.0, 0.0])
    output = torch.tensor([1.03, 5.03, -5.06, 0.019])
    s = summarize_errors(output, reference)
    # 0.03 at |ref| 1 fails both parts; 0.03 at 5 passes the rel part (0.05);
    # 0.06 at 5 fails both; 0.019 at 0 passes the abs part
    assert s.outside == 2 and s.total == 4 and s.finite
    assert s.max_abs == pytest.approx(0.06, abs=1e-6)
    assert s.mean_abs == pytest.approx((0.03 + 0.03 + 0.06 + 0.019) / 4, abs=1e-6)
    bad = summarize_errors(torch.tensor([1.0, float("nan"), -5.0, 0.0]), reference)
    assert not bad.finite and bad.outside == 1 and bad.max_abs == float("inf")


def _noisy(exact, scale, seed, dtype=torch.bfloat16):
    generator = torch.Generator().manual_seed(seed)
    return (exact + scale * torch.randn(exact.shape, generator=generator)).to(dtype)


def test_model_parity_compares_both_pipelines_with_fp32():
    from oracle.compare import model_parity

    generator = torch.Generator().manual_seed(0)
    exact = torch.randn(2, 64, 128, generator=generator) * 3
    reference_path = _noisy(exact, 0.01, 1)
    # an independent pipeline with the same noise level passes; so does the
    # reference path itself and a more accurate candidate
    assert model_parity(exact, reference_path, _noisy(exact, 0.01, 2)).passed
    assert model_parity(exact, reference_path, reference_path).passed
    assert model_parity(exact, reference_path, exact.to(torch.bfloat16)).passed
    # twice the noise, a 1% fraction of far-off elements, a bias or a NaN fail
    assert not model_parity(exact, reference_path, _noisy(exact, 0.02, 2)).passed
    far = reference_path.float().clone()
    far.view(-1)[: far.numel() // 100] += 0.5
    assert not model_parity(exact, reference_path, far.to(torch.bfloat16)).passed
    assert not model_parity(exact, reference_path, (exact + 0.05).to(torch.bfloat16)).passed
    nan = reference_path.float().clone()
    nan.view(-1)[7] = float("nan")
    assert not model_parity(exact, reference_path, nan).passed
    # the candidate is measured against fp32, not against the reference path:
    # an accurate reference path makes a noisy candidate fail
    accurate = exact.to(torch.bfloat16)
    assert not model_parity(exact, accurate, _noisy(exact, 0.01, 2)).passed
    # the elementwise north-star gate is reported on both sides
    parity = model_parity(exact, reference_path, _noisy(exact, 0.01, 2))
    assert parity.strict_vs_reference_path == parity.candidate_vs_reference_path.passed
    assert "elementwise 2e-2/1e-2 gate" in parity.summary()


def test_launch_search_gate_is_the_model_parity_rule():
    from autotune.accuracy import no_less_accurate
    from autotune.hip_launch_search import no_less_accurate as search_gate
    from oracle.compare import model_parity

    assert search_gate is no_less_accurate
    generator = torch.Generator().manual_seed(3)
    exact = torch.randn(2, 32, 64, generator=generator) * 2
    incumbent = _noisy(exact, 0.01, 4)
    for candidate in (_noisy(exact, 0.01, 5), _noisy(exact, 0.015, 5), _noisy(exact, 0.03, 5)):
        assert no_less_accurate(candidate, incumbent, exact) == model_parity(exact, incumbent, candidate).passed


def test_gate_ratio_is_at_most_one_exactly_when_the_gate_passes():
    from autotune.accuracy import gate_ratio, summarize_errors

    reference = torch.tensor([1.0, 5.0, -5.0, 0.0])
    # allowances: max(0.02, 0.01 |ref|) = 0.02, 0.05, 0.05, 0.02
    output = torch.tensor([1.01, 5.03, -5.04, 0.005])
    assert gate_ratio(output, reference, atol=0.02, rtol=0.01) == pytest.approx(0.8, rel=1e-4)
    assert summarize_errors(output, reference).outside == 0
    failing = torch.tensor([1.03, 5.0, -5.0, 0.0])  # 0.03 / 0.02
    assert gate_ratio(failing, reference, atol=0.02, rtol=0.01) == pytest.approx(1.5, rel=1e-4)
    assert summarize_errors(failing, reference).outside == 1
    # a zero allowance: exact elements count 0, others infinity
    assert gate_ratio(torch.zeros(3), torch.zeros(3), atol=0.0, rtol=0.01) == 0.0
    assert gate_ratio(torch.tensor([1e-6]), torch.zeros(1), atol=0.0, rtol=0.01) == float("inf")
    assert gate_ratio(torch.tensor([float("nan")]), torch.ones(1), atol=0.02, rtol=0.01) == float("inf")
    generator = torch.Generator().manual_seed(9)
    ref = torch.randn(1000, generator=generator)
    out = ref + 0.03 * torch.randn(1000, generator=generator)
    ratio = gate_ratio(out, ref, atol=0.02, rtol=0.01)
    assert (ratio <= 1.0) == (summarize_errors(out, ref).outside == 0)
