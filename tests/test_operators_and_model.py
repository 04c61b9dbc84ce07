"""Portable operators and the plugin model on the CPU (no GPU needed)."""

from __future__ import annotations

import math

import pytest
import torch

from oracle.compare import parity_gate
from oracle.forward import TransformerConfig, default_init_weights, forward, generate_input
from solution.config import hip_config, portable_config, portable_streamed_config
from solution.operators import (
    can_split_qkv,
    can_use_causal_sdpa,
    can_use_residual_add,
    causal_sdpa,
    reference_causal_attention,
    residual_add,
    split_qkv,
)
from solution.plan_builder import ConfigRejectedError
from solution.transformer import UserOptimizedTransformer, copy_model_weights


class _StateSource(torch.nn.Module):
    """Minimal stand-in for the official model: exposes a state dict."""

    def __init__(self, tensors):
        super().__init__()
        self._tensors = tensors

    def state_dict(self, *args, **kwargs):
        return dict(self._tensors)


def test_split_qkv_is_a_zero_copy_view():
    """Restates tests/solution/test_causal_operators.py:19-27 of the reference."""

    packed = torch.arange(2 * 5 * 3 * 8, dtype=torch.float32).view(2, 5, 24)
    query, key, value = split_qkv(packed, num_heads=2)
    assert query.shape == key.shape == value.shape == (2, 2, 5, 4)
    assert query.untyped_storage().data_ptr() == packed.untyped_storage().data_ptr()
    assert query.stride() == (120, 4, 24, 1)
    assert torch.equal(key[1, 1, 3], packed[1, 3, 12:16])
    assert can_split_qkv(packed, num_heads=2) and not can_split_qkv(packed, num_heads=3)
    assert all(t.is_contiguous() for t in split_qkv(packed, 2, contiguous=True))


def test_causal_sdpa_matches_explicit_float32_math():
    generator = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(2, 4, 7, 8, generator=generator) for _ in range(3))
    scores = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(8)
    scores.masked_fill_(torch.triu(torch.ones(7, 7, dtype=torch.bool), diagonal=1), float("-inf"))
    expected = torch.matmul(torch.softmax(scores, dim=-1), v)
    torch.testing.assert_close(causal_sdpa(q, k, v), expected, rtol=2e-5, atol=2e-6)
    assert not can_use_causal_sdpa(q.bfloat16(), k.bfloat16(), v.bfloat16())


def test_reference_attention_with_key_mask_matches_full_order():
    generator = torch.Generator().manual_seed(19)
    q, k, v = (torch.randn(2, 2, 9, 4, generator=generator) for _ in range(3))
    valid = torch.tensor([[True] * 5 + [False] * 4, [True] * 7 + [False] * 2])
    actual = reference_causal_attention(q, k, v, valid, query_block_size=4)
    scores = torch.matmul(q, k.transpose(-2, -1)) / 2.0
    scores.masked_fill_(torch.ones(9, 9, dtype=torch.bool).triu(diagonal=1), float("-inf"))
    scores.masked_fill_((~valid)[:, None, None, :], float("-inf"))
    torch.testing.assert_close(actual, torch.matmul(torch.softmax(scores, dim=-1), v))
    with pytest.raises(ValueError):
        reference_causal_attention(q, k, v, query_block_size=0)


def test_residual_add_masks_only_invalid_query_tokens():
    value = torch.ones(2, 3, 4)
    valid = torch.tensor([[True, False, True], [False, True, True]])
    out = residual_add(value, torch.full_like(value, 2.0), valid)
    assert can_use_residual_add(value, value, valid)
    assert torch.all(out[valid] == 3.0) and torch.all(out[~valid] == 0.0)


def _model(config, state, dtype=torch.float32):
    model = UserOptimizedTransformer(config)
    copy_model_weights(_StateSource(state), model)
    return model.to(dtype).eval()


def test_copy_model_weights_packs_qkv_and_is_strict():
    config = TransformerConfig(1, 8, 64, 4, 128, 2, True)
    state = default_init_weights(config, seed=5)
    model = _model(config, state)
    packed = model.layers[1].attention.qkv_proj.weight
    expected = torch.cat([state[f"layers.1.attention.{n}_proj.weight"] for n in "qkv"])
    assert torch.equal(packed, expected)
    broken = dict(state)
    broken.pop("layers.0.ffn_in.bias")
    with pytest.raises(RuntimeError, match="strict weight mapping failed"):
        copy_model_weights(_StateSource(broken), UserOptimizedTransformer(config))
    extra = dict(state, **{"unused.weight": torch.zeros(1)})
    with pytest.warns(RuntimeWarning, match="unused source keys"):
        copy_model_weights(_StateSource(extra), UserOptimizedTransformer(config), strict=False)


@pytest.mark.parametrize("config_factory", [portable_config, lambda: portable_streamed_config(microbatch_size=1)])
def test_portable_model_equals_the_oracle_on_config1(config_factory):
    """BASELINE config 1 (CPU fp32): the plugin model with the reference-order
    program reproduces the oracle forward, and the observed path equals the
    plan's expected trace."""

    config = TransformerConfig(2, 128, 256, 4, 1024, 2, True)
    state = default_init_weights(config, seed=1234)
    model = _model(config, state)
    chosen = config_factory()
    if chosen.schedule.runtime.value == "streamed":
        with pytest.raises(ConfigRejectedError, match="requires_cuda"):
            model.configure_execution(config=chosen)
        return
    model.configure_execution(config=chosen)
    model.set_execution_observation(True)
    x = generate_input(config, seed=1234)
    with torch.inference_mode():
        output = model(x)
    reference = forward(state, x, config)
    assert parity_gate(reference, output, torch.float32).passed
    description = model.describe_execution_path()
    expected = description["expected_execution_signature"]
    observed = description["observed_execution_signature"]
    assert observed["complete"] and observed == expected


def test_default_config_on_cpu_is_portable_and_all_valid_mask_collapses():
    config = TransformerConfig(2, 16, 64, 4, 128, 1, True)
    state = default_init_weights(config, seed=2)
    model = _model(config, state)
    x = generate_input(config, seed=2)
    with torch.inference_mode():
        plain = model(x)
        masked = model(x, torch.ones(2, 16, dtype=torch.bool))
    assert torch.equal(plain, masked)
    assert model.describe_execution_path()["planned_config_id"] == portable_config().config_id


def test_hip_config_is_rejected_on_cpu_without_fallback():
    config = TransformerConfig(2, 16, 64, 4, 128, 1, True)
    model = _model(config, default_init_weights(config, seed=2))
    with pytest.raises(ConfigRejectedError, match="program.attention"):
        model.configure_execution(config=hip_config())
